"""Decoder-layer ops on the gfx950 kernels (the layers the reference takes
from FlashInfer, Triton and torch: python/aios/layers/norm.py:10-40,
layers/activation.py:9-12, layers/attention.py:11-16, the q/k norm of
models/qwen3.py:65-66 and the Block-AttnRes depth mixer,
kernel/attnres.py:130-223).

``HipOps`` is the op set the decoder uses on the GPU; every call goes
through the C ABI of libaios_attn.so and fails loudly without it.
"""
from __future__ import annotations

import torch

from aios_amd import _lib


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_rows(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or not t.is_cuda or t.ndim != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D bfloat16 GPU tensor with contiguous rows")


class HipOps:
    """RMSNorm, residual-add RMSNorm, q/k RMSNorm + RoPE, SiLU-and-mul, and
    the projections (few-row GEMM kernel for decode-sized inputs, the
    library GEMM for larger ones)."""

    # The decoder may hand an appending decode batch's raw q/k projections to
    # the attention backend, which applies the q/k RMSNorm + RoPE of
    # qk_norm_rope inside the decode launch.
    rope_in_decode = True

    @staticmethod
    def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        rows, k = x.shape
        n = weight.shape[0]
        if (rows > 64 or n % 16 or k % 128 or x.dtype != torch.bfloat16
                or weight.dtype != torch.bfloat16 or x.stride(1) != 1 or weight.stride(1) != 1
                or x.stride(0) % 8 or weight.stride(0) % 8):
            return torch.nn.functional.linear(x, weight)
        if rows == 0:
            return x.new_empty(0, n)
        y = torch.empty(rows, n, dtype=x.dtype, device=x.device)
        _lib.check(_lib.lib().aios_linear_rows(x.data_ptr(), x.stride(0), weight.data_ptr(),
                                               weight.stride(0), y.data_ptr(), y.stride(0), rows,
                                               n, k, _stream(x)), "aios_linear_rows")
        return y

    @staticmethod
    def _rows_ok(x: torch.Tensor, weight: torch.Tensor, k: int) -> bool:
        return (x.shape[0] <= 64 and weight.shape[0] % 16 == 0 and k % 128 == 0
                and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
                and x.stride(1) == 1 and weight.stride(1) == 1 and x.stride(0) % 8 == 0
                and weight.stride(0) % 8 == 0 and x.shape[0] > 0)

    def add_rmsnorm_linear(self, h: torch.Tensor, residual: torch.Tensor | None,
                           norm_weight: torch.Tensor, eps: float, weight: torch.Tensor,
                           silu: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """RMSNormFused then a projection (norm.py:24-40): returns
        (linear(RMSNorm(h + residual) * w), h + residual); with no residual the
        new residual is h itself.  silu=True: weight is the merged gate/up
        matrix and the projection is followed by silu_and_mul
        (activation.py:9-12)."""
        rows, k = h.shape
        n = weight.shape[0] // 2 if silu else weight.shape[0]
        # The prologue keeps (K/128) x (16-row tiles) normalised fragments in
        # registers, at most 8: more rows than one launch holds run as row
        # chunks (each re-reading the weights, mostly from L2) rather than
        # as separate norm, projection and activation launches.
        frags = (k // 4) // 32
        chunk = 16 * (8 // frags) if 1 <= frags <= 8 else 0
        if chunk and self._rows_ok(h, weight, k) and n % 16 == 0 and \
                (residual is None or (residual.stride(1) == 1 and residual.stride(0) % 8 == 0)):
            y = torch.empty(rows, n, dtype=h.dtype, device=h.device)
            new_res = torch.empty_like(h) if residual is not None else h
            lib = _lib.lib()
            for r0 in range(0, rows, chunk):
                m = min(chunk, rows - r0)
                _lib.check(lib.aios_linear_rows_ex(
                    h[r0:].data_ptr(), h.stride(0), weight.data_ptr(), weight.stride(0),
                    y[r0:].data_ptr(), y.stride(0), m, n, k, _lib.PROLOGUE_ADD_RMSNORM,
                    residual[r0:].data_ptr() if residual is not None else None,
                    residual.stride(0) if residual is not None else 0, norm_weight.data_ptr(),
                    eps, new_res[r0:].data_ptr() if residual is not None else None,
                    new_res.stride(0) if residual is not None else 0,
                    _lib.EPILOGUE_SILU_MUL if silu else _lib.EPILOGUE_NONE, _stream(h)),
                    "aios_linear_rows_ex")
            return y, new_res
        if residual is None:
            x, residual = self.rmsnorm(h, norm_weight, eps), h
        else:  # (the inputs are left unchanged, as on the folded path)
            x, residual = self.fused_add_rmsnorm(h.clone(), residual.clone(), norm_weight, eps)
        y = self.linear(x, weight)
        return (self.silu_and_mul(y) if silu else y), residual

    @staticmethod
    def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
        _check_rows(x, "x")
        out = torch.empty_like(x)
        _lib.check(_lib.lib().aios_rmsnorm(x.data_ptr(), x.stride(0), None, 0, weight.data_ptr(),
                                           out.data_ptr(), out.stride(0), x.shape[0], x.shape[1],
                                           eps, _stream(x)), "aios_rmsnorm")
        return out

    @staticmethod
    def fused_add_rmsnorm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                          eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        """residual <- x + residual; x <- RMSNorm(residual) * weight (both in place)."""
        _check_rows(x, "x")
        _check_rows(residual, "residual")
        if x.shape != residual.shape:
            raise ValueError("x and residual must have the same shape")
        _lib.check(_lib.lib().aios_rmsnorm(x.data_ptr(), x.stride(0), residual.data_ptr(),
                                           residual.stride(0), weight.data_ptr(), x.data_ptr(),
                                           x.stride(0), x.shape[0], x.shape[1], eps, _stream(x)),
                   "aios_rmsnorm")
        return x, residual

    @staticmethod
    def qk_norm_rope(qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                     cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                     num_qo_heads: int, num_kv_heads: int, head_dim: int,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor]:
        """q, k = RoPE(RMSNorm_head(q)), RoPE(RMSNorm_head(k)) from qkv rows."""
        _check_rows(qkv, "qkv")
        if positions.dtype != torch.int32 or positions.numel() != qkv.shape[0]:
            raise ValueError("positions must be int32 with one entry per token")
        if cos.dtype != torch.float32 or cos.shape != sin.shape or cos.shape[1] != head_dim:
            raise ValueError("cos/sin tables must be float32 [positions, head_dim]")
        t = qkv.shape[0]
        q = torch.empty(t, num_qo_heads, head_dim, dtype=qkv.dtype, device=qkv.device)
        k = torch.empty(t, num_kv_heads, head_dim, dtype=qkv.dtype, device=qkv.device)
        _lib.check(_lib.lib().aios_qk_norm_rope(
            qkv.data_ptr(), qkv.stride(0), t, num_qo_heads, num_kv_heads, head_dim,
            q_weight.data_ptr(), k_weight.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
            positions.contiguous().data_ptr(), q.data_ptr(), k.data_ptr(), eps, _stream(qkv)),
            "aios_qk_norm_rope")
        return q, k

    @staticmethod
    def attnres_mix(bank: torch.Tensor, partial: torch.Tensor | None,
                    weighted_query: torch.Tensor, eps: float) -> torch.Tensor:
        """Depth mix of bank [S, N, D] (+ partial as the last source)."""
        from aios_amd.kernel import attnres_mix

        return attnres_mix(bank, partial, weighted_query, eps)

    @staticmethod
    def attnres_mix_step(bank: torch.Tensor, partial: torch.Tensor | None, delta: torch.Tensor,
                         weighted_query: torch.Tensor, eps: float,
                         partial_out: torch.Tensor) -> torch.Tensor:
        """partial_out <- partial + delta, then the mix with it as the last source."""
        from aios_amd.kernel import attnres_mix_step

        return attnres_mix_step(bank, partial, delta, weighted_query, eps, partial_out)

    @staticmethod
    def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
        _check_rows(x, "x")
        inter = x.shape[1] // 2
        out = torch.empty(x.shape[0], inter, dtype=x.dtype, device=x.device)
        _lib.check(_lib.lib().aios_silu_mul(x.data_ptr(), x.stride(0), x.shape[0], inter,
                                            out.data_ptr(), out.stride(0), _stream(x)),
                   "aios_silu_mul")
        return out
