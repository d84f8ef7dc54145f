"""Block-AttnRes depth mixer entry points (HIP kernel behind the C ABI).

``attnres_mix`` keeps the signature, validation and error messages of the
reference's ``triton_attnres_mix`` (python/aios/kernel/attnres.py:130-223),
so a mixer backend can call either.  It runs one launch
(``aios_attnres_mix``) that reads the bank once.

``attnres_mix_step`` is the decoder's fused form: the running partial is
formed in the same launch as ``partial + delta`` (the adds of
python/aios/models/minimind_ime.py:233-252) and stored to ``partial_out``.
"""
from __future__ import annotations

import torch

from aios_amd import _lib


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_bank(bank: torch.Tensor) -> tuple[int, int, int]:
    if not bank.is_cuda:
        raise ValueError("AttnRes mix requires GPU tensors")
    if bank.ndim != 3:
        raise ValueError("bank must have shape [S,N,D]")
    if not bank.is_contiguous():
        raise ValueError("bank must be contiguous for the kernel's pointer layout")
    s, n, d = bank.shape
    if s < 1 or n < 1 or d < 1:
        raise ValueError("bank dimensions must be positive")
    if bank.dtype != torch.bfloat16:
        raise ValueError("the HIP AttnRes mix is built for bfloat16 banks")
    return s, n, d


def _check_plane(t: torch.Tensor, bank: torch.Tensor, name: str) -> None:
    if t.shape != bank.shape[1:]:
        raise ValueError(f"{name} must match bank [N,D]")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.dtype != bank.dtype or t.device != bank.device:
        raise ValueError(f"{name} must match bank dtype/device")


def _check_query(weighted_query: torch.Tensor, hidden: int, bank: torch.Tensor) -> None:
    if weighted_query.shape != (hidden,):
        raise ValueError("weighted_query must match hidden size")
    if not weighted_query.is_contiguous():
        raise ValueError("weighted_query must be contiguous")
    if weighted_query.dtype != torch.float32 or weighted_query.device != bank.device:
        raise ValueError("weighted_query must be float32 on the bank device")


def _scores(score_buffer, total: int, n: int, bank: torch.Tensor):
    if score_buffer is None:
        return None
    if score_buffer.dtype != torch.float32 or score_buffer.device != bank.device:
        raise ValueError("score_buffer must be GPU float32 on bank device")
    if (score_buffer.shape[0] < total or score_buffer.shape[1] != n
            or not score_buffer.is_contiguous()):
        raise ValueError("score_buffer must be contiguous [capacity_sources, num_tokens]")
    return score_buffer[:total]


def _output(output_buffer, bank: torch.Tensor) -> torch.Tensor:
    if output_buffer is None:
        return torch.empty_like(bank[0])
    if output_buffer.shape != bank.shape[1:]:
        raise ValueError("output_buffer must match bank [N,D]")
    if output_buffer.dtype != bank.dtype or output_buffer.device != bank.device:
        raise ValueError("output_buffer must match bank dtype/device")
    if not output_buffer.is_contiguous():
        raise ValueError("output_buffer must be contiguous")
    return output_buffer


def attnres_mix(
    bank: torch.Tensor,
    partial: torch.Tensor | None,
    weighted_query: torch.Tensor,
    eps: float,
    *,
    score_buffer: torch.Tensor | None = None,
    output_buffer: torch.Tensor | None = None,
) -> torch.Tensor:
    """Depth-softmax mix of ``bank`` (and ``partial`` as the last source):
    fp32 RMS scores, bf16 weights, fp32 weighted sum, bf16 output."""
    s, n, d = _check_bank(bank)
    if partial is not None:
        _check_plane(partial, bank, "partial")
    _check_query(weighted_query, d, bank)
    total = s + int(partial is not None)
    scores = _scores(score_buffer, total, n, bank)
    out = _output(output_buffer, bank)
    _lib.check(_lib.lib().aios_attnres_mix(
        bank.data_ptr(), s, n, d, partial.data_ptr() if partial is not None else None,
        weighted_query.data_ptr(), float(eps), scores.data_ptr() if scores is not None else None,
        out.data_ptr(), _stream(bank)), "aios_attnres_mix")
    return out


def attnres_mix_step(
    bank: torch.Tensor,
    partial: torch.Tensor | None,
    delta: torch.Tensor,
    weighted_query: torch.Tensor,
    eps: float,
    partial_out: torch.Tensor,
    *,
    output_buffer: torch.Tensor | None = None,
) -> torch.Tensor:
    """``partial_out <- partial + delta`` (``delta`` when partial is None),
    then the mix of ``bank`` with that partial as the last source."""
    s, n, d = _check_bank(bank)
    if partial is not None:
        _check_plane(partial, bank, "partial")
    _check_plane(delta, bank, "delta")
    _check_plane(partial_out, bank, "partial_out")
    _check_query(weighted_query, d, bank)
    out = _output(output_buffer, bank)
    _lib.check(_lib.lib().aios_attnres_mix_ex(
        bank.data_ptr(), s, n, d, partial.data_ptr() if partial is not None else None,
        delta.data_ptr(), partial_out.data_ptr(), weighted_query.data_ptr(), float(eps), None,
        out.data_ptr(), _stream(bank)), "aios_attnres_mix_ex")
    return out
