"""Stateless candidate sampling on the gfx950 kernels (the interface of
python/aios/engine/sample.py: ``stateless_uniforms`` and
``Sampler.sample_with_logprobs``).

``stateless_uniforms`` computes the SplitMix64 uniforms on the device
(``aios_stateless_uniforms``), keyed by (candidate seed, token step), so a
candidate keeps its stream wherever its row sits in the batch.
``Sampler.sample_with_logprobs`` is one launch of ``aios_sample`` per call:
temperature / top-k / top-p on a sampling copy with forbidden ids at -inf,
the token chosen by the candidate's uniform, and the raw log-probability of
the unmodified distribution.  ``sample_step`` is the same launch with the
step index read on the device, for graph-replayed decode loops.

Ties in the top-k order go to the lower token id.  Without ``uniforms`` the
uniforms are drawn with ``torch.rand`` (the reference uses
``torch.multinomial`` there; that stream is not reproduced).
"""
from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from aios_amd import _lib
from aios_amd.core import SamplingParams

_NO_STEP_LIMIT = 2**31 - 1


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def stateless_uniforms(candidate_seeds: Sequence[int] | torch.Tensor, steps: int,
                       device: torch.device) -> torch.Tensor:
    """``(rows, steps)`` float32 uniforms, one independent stream per seed."""
    if steps < 1:
        raise ValueError("steps must be positive")
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("stateless_uniforms runs on the GPU")
    seeds = torch.as_tensor(candidate_seeds, dtype=torch.int64)
    if seeds.device != device:
        seeds = seeds.to(device)
    seeds = seeds.contiguous()
    out = torch.empty((seeds.numel(), steps), dtype=torch.float32, device=device)
    _lib.check(_lib.lib().aios_stateless_uniforms(seeds.data_ptr(), seeds.numel(), steps,
                                                  out.data_ptr(), _stream(out)),
               "aios_stateless_uniforms")
    return out


def _check_logits(logits: torch.Tensor) -> None:
    if logits.ndim != 2 or logits.stride(1) != 1 or not logits.is_cuda:
        raise ValueError("logits must be a 2-D GPU tensor with contiguous rows")
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("logits must be bfloat16 or float32")


def sample_step(logits: torch.Tensor, params: SamplingParams, uniforms: torch.Tensor,
                step: torch.Tensor, forbidden_ids: torch.Tensor | None = None,
                forbid_before_step: int = _NO_STEP_LIMIT,
                forbidden_by_row: torch.Tensor | None = None,
                out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """Graph-safe launch: row r uses ``uniforms[r, step]`` with ``step`` a
    device int64 scalar; ``forbidden_ids`` (device int32) apply while
    ``step < forbid_before_step``.  Returns (tokens int64 [rows], raw
    log-probs fp32 [rows])."""
    _check_logits(logits)
    rows, vocab = logits.shape
    if uniforms.dtype != torch.float32 or uniforms.ndim != 2 or uniforms.shape[0] != rows \
            or uniforms.stride(1) != 1:
        raise ValueError("uniforms must be float32 [rows, steps] with contiguous rows")
    if step.dtype != torch.int64 or step.numel() != 1:
        raise ValueError("step must be a one-element int64 tensor")
    if forbidden_by_row is not None and (
            forbidden_by_row.dtype != torch.int64 or forbidden_by_row.ndim != 2
            or forbidden_by_row.shape[0] != rows or not forbidden_by_row.is_contiguous()):
        raise ValueError("forbidden_by_row must be contiguous int64 [rows, n]")
    tok, lp = out if out is not None else (
        torch.empty(rows, dtype=torch.int64, device=logits.device),
        torch.empty(rows, dtype=torch.float32, device=logits.device))
    nf = 0 if forbidden_ids is None else forbidden_ids.numel()
    nr = 0 if forbidden_by_row is None else forbidden_by_row.shape[1]
    _lib.check(_lib.lib().aios_sample(
        logits.data_ptr(), logits.stride(0), rows, vocab, logits.element_size(),
        float(params.temperature), int(params.top_k), float(params.top_p),
        uniforms.data_ptr(), uniforms.stride(0), uniforms.shape[1], step.data_ptr(),
        forbidden_ids.data_ptr() if nf else None, nf, int(forbid_before_step),
        forbidden_by_row.data_ptr() if nr else None, nr, tok.data_ptr(), lp.data_ptr(),
        _stream(logits)), "aios_sample")
    return tok, lp


@dataclass
class Sampler:
    """engine/sample.py:50-160 on the sampling kernel."""

    sampling_params: SamplingParams

    def sample_with_logprobs(
        self,
        logits: torch.Tensor,
        *,
        generator: torch.Generator | None = None,
        uniforms: torch.Tensor | None = None,
        forbidden_token_ids: Sequence[int] = (),
        forbidden_token_ids_by_row: torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """(token ids [rows, 1], raw log-probs [rows, 1]) of 2-D logits."""
        if generator is not None and uniforms is not None:
            raise ValueError("generator and uniforms are mutually exclusive")
        _check_logits(logits)
        rows, vocab = logits.shape
        blocked = sorted({int(t) for t in forbidden_token_ids})
        invalid = [t for t in blocked if t < 0 or t >= vocab]
        if invalid:
            raise ValueError(f"forbidden token ids are outside the vocabulary: {invalid}")
        by_row = None
        if forbidden_token_ids_by_row is not None:
            f = forbidden_token_ids_by_row
            if f.ndim != 2 or f.shape[0] != rows:
                raise ValueError("forbidden_token_ids_by_row must have shape [batch, count]")
            if f.device.type == "cpu" and not bool(((f >= 0) & (f < vocab)).all().item()):
                raise ValueError("row-specific forbidden token ids are outside the vocabulary")
            by_row = f.to(device=logits.device, dtype=torch.int64).contiguous()
            if by_row.shape[1] == 0:
                by_row = None
        p = self.sampling_params
        if p.is_greedy:
            u = torch.full((rows, 1), 0.5, dtype=torch.float32, device=logits.device)
        elif uniforms is None:
            u = torch.rand((rows, 1), generator=generator, device=logits.device)
        else:
            if tuple(uniforms.shape) != (rows,):
                raise ValueError("uniforms must match the sampling batch dimensions: "
                                 f"expected {(rows,)}, got {tuple(uniforms.shape)}")
            u = uniforms.to(device=logits.device, dtype=torch.float32).reshape(rows, 1).contiguous()
        ids = (torch.tensor(blocked, dtype=torch.int32, device=logits.device) if blocked else None)
        step = torch.zeros(1, dtype=torch.int64, device=logits.device)
        tok, lp = sample_step(logits, p, u, step, ids, _NO_STEP_LIMIT, by_row)
        return tok[:, None], lp[:, None]

    def sample(self, logits: torch.Tensor) -> torch.Tensor:
        return self.sample_with_logprobs(logits)[0]
