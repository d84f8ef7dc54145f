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
