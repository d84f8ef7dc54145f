"""Greedy selection kernel (aios_greedy_select) vs torch argmax / log_softmax.

The token must equal torch's argmax of the logits as stored (first index of
the maximum, sample.py:115-117) bit for bit; the log-prob must match
log_softmax of the fp32-widened logits (sample.py:73) computed in float64.
"""
from __future__ import annotations

import pytest
import torch

from aios_amd.paged import greedy_select

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(8, 6400), (8, 151936), (3, 1), (5, 7), (24, 16384)])
def test_greedy_matches_torch(dtype, rows, vocab):
    g = torch.Generator(device="cuda").manual_seed(rows * 7 + vocab)
    x = (torch.randn(rows, vocab, generator=g, device="cuda") * 3.0).to(dtype)
    tok, lp = greedy_select(x)
    ref_tok = x.argmax(dim=-1)
    assert torch.equal(tok, ref_tok)
    ref_lp = torch.log_softmax(x.double(), dim=-1).gather(1, ref_tok[:, None]).squeeze(1)
    torch.testing.assert_close(lp.double(), ref_lp, atol=2e-5, rtol=1e-5)


def test_ties_take_the_first_index_and_strided_rows():
    x = torch.zeros(4, 1000, dtype=torch.bfloat16, device="cuda")
    x[0, [5, 700]] = 2.0
    x[1, [999, 3]] = 1.0
    x[2] = -1.0  # all equal: index 0
    x[3, 513] = 7.0
    wide = torch.zeros(4, 1100, dtype=torch.bfloat16, device="cuda")
    wide[:, :1000] = x
    wide[:, 1000:] = 100.0  # outside the row's vocab: never read
    tok, lp = greedy_select(wide[:, :1000])
    assert tok.tolist() == [5, 3, 0, 513]
    ref = torch.log_softmax(x.double(), -1).gather(1, tok[:, None]).squeeze(1)
    torch.testing.assert_close(lp.double(), ref, atol=2e-5, rtol=1e-5)
    assert abs(lp[2].item() - (-torch.log(torch.tensor(1000.0)).item())) < 1e-4
