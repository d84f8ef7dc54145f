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


# --- stateless sampling (aios_sample, aios_stateless_uniforms) ---------------

import numpy as np  # noqa: E402

from aios_amd.core import SamplingParams  # noqa: E402
from aios_amd.sample import Sampler, sample_step, stateless_uniforms  # noqa: E402
from oracle import sampling as osamp  # noqa: E402


def test_stateless_uniforms_match_oracle_bitwise():
    seeds = [20260814 + i for i in range(8)] + [0, 1, 2**62 + 12345, 987654321987]
    got = stateless_uniforms(seeds, 24, torch.device("cuda")).cpu().numpy()
    assert np.array_equal(got, osamp.stateless_uniforms(seeds, 24))


def _check_rows(x, params, u, forbidden=(), by_row=None):
    """Kernel tokens vs the oracle: equal ids wherever u sits farther than
    TOL from a cumulative boundary (fp32 sums in another order may land on
    the neighbour there: 1e-5 for top-k, 2e-4 for the every-id mode that
    sums a whole vocabulary), else the id's position must bracket u within
    TOL; where top_p itself sits on a cumulative sum the id must be one of
    the candidates.  The raw log-prob of the chosen id within 2e-5.  Returns
    the number of rows whose top-p cut was ambiguous."""
    s = Sampler(params)
    tok, lp = s.sample_with_logprobs(x, uniforms=u, forbidden_token_ids=forbidden,
                                     forbidden_token_ids_by_row=by_row)
    tok, lp = tok[:, 0].cpu(), lp[:, 0].cpu()
    xs = x.float().cpu().numpy()
    tol = 2e-4 if params.top_k <= 0 and not params.is_greedy else 1e-5
    ambiguous = 0
    for r in range(x.shape[0]):
        fb = list(forbidden) + ([] if by_row is None else by_row[r].tolist())
        want, _, d = osamp.sample_row(xs[r], params.temperature, params.top_k, params.top_p,
                                      float(u[r]), fb, detail=True)
        t = int(tok[r])
        assert t not in set(fb)
        order, cum = d["order"], d["cum"]
        if d["cut_margin"] <= tol:
            # top_p sits on a cumulative sum: the cut may keep one more or
            # one fewer candidate; the id is one of the top-k
            assert t in set(order.tolist()), (r, t)
            ambiguous += 1
        elif d["u_margin"] > tol:
            assert t == want, (r, t, want)
        else:
            # u on a boundary: the id's position brackets u within tol
            pos = int(np.nonzero(order == t)[0][0])
            lo = cum[pos - 1] if pos > 0 else 0.0
            assert lo - tol < float(u[r]), (r, t, want)
            assert float(u[r]) <= cum[pos] + tol or pos == len(cum) - 1, (r, t, want)
        raw = xs[r].astype(np.float64)
        ref_lp = raw[t] - raw.max() - np.log(np.exp(raw - raw.max()).sum())
        assert abs(float(lp[r]) - ref_lp) < 2e-5 * max(1.0, abs(ref_lp))
    return ambiguous


PARAMS = [
    SamplingParams(temperature=0.35, top_k=50, top_p=0.9),    # the IME first round
    SamplingParams(temperature=0.75, top_k=96, top_p=0.95),   # the first refill round
    SamplingParams(temperature=0.95, top_k=160, top_p=0.95),
    SamplingParams(temperature=1.0, top_k=1024, top_p=1.0),
    SamplingParams(temperature=0.8, top_k=-1, top_p=1.0),      # every id, id order
    SamplingParams(temperature=0.0),                           # greedy
    SamplingParams(temperature=0.7, top_k=1),                  # greedy by top_k
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("vocab", [6400, 151936, 37, 4100, 16384])
@pytest.mark.parametrize("pi", range(len(PARAMS)))
def test_sample_matches_oracle(dtype, vocab, pi):
    params = PARAMS[pi]
    rows = 24
    g = torch.Generator(device="cuda").manual_seed(vocab + 31 * pi)
    stride = (vocab + 7) // 8 * 8
    full = (torch.randn(rows, stride, generator=g, device="cuda") * 3.0).to(dtype)
    x = full[:, :vocab]
    u = stateless_uniforms([1000 * pi + r for r in range(rows)], 1, torch.device("cuda"))[:, 0]
    assert _check_rows(x, params, u) <= 2  # rows whose cut top_p happens to sit on


def test_sample_ties_and_forbidden():
    """Heavily tied bf16 logits (few distinct values) and forbidden ids, both
    the global list and per row (including duplicates and the pad-id style
    repeats the reference scatters)."""
    rows, vocab = 16, 6400
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randint(-4, 4, (rows, vocab), generator=g, device="cuda").to(torch.bfloat16) * 0.5
    x[:, 17] = 3.0
    x[:, 4000] = 3.0
    u = stateless_uniforms(list(range(rows)), 1, torch.device("cuda"))[:, 0]
    by_row = torch.tensor([[17, 0, 0], [4000, 4000, 1]] * (rows // 2), dtype=torch.int64,
                          device="cuda")
    for params in (SamplingParams(temperature=0.5, top_k=50, top_p=0.9),
                   SamplingParams(temperature=1.0, top_k=300, top_p=1.0),
                   SamplingParams(temperature=0.0)):
        _check_rows(x, params, u, forbidden=(5, 6, 17), by_row=by_row)
    # greedy with every maximum forbidden: the next value, lowest id
    tok, _ = Sampler(SamplingParams()).sample_with_logprobs(x[:2], forbidden_token_ids=(17, 4000))
    want = [int(((x[r].float() == 1.5).nonzero()[0]).item()) for r in range(2)]
    assert tok[:, 0].tolist() == want


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sample_ties_beyond_the_candidate_buffer(dtype):
    """Four distinct values over 16384 ids: about 4096 ids tie at each value,
    so the ids at or above the k-th value overflow the row-resident kernel's
    2048-entry candidate buffer and the exact k-th value key and id cut are
    found by bisection; the lowest tied ids must be taken.  Forbidden ids
    among the top ties shift the cut."""
    rows, vocab = 8, 16384
    g = torch.Generator(device="cuda").manual_seed(11)
    x = (torch.randint(0, 4, (rows, vocab), generator=g, device="cuda").to(torch.float32) * 0.5).to(dtype)
    u = stateless_uniforms([500 + r for r in range(rows)], 1, torch.device("cuda"))[:, 0]
    top = [int((x[r].float() == 1.5).nonzero()[0].item()) for r in range(rows)]
    by_row = torch.tensor([[t, t + 1] for t in top], dtype=torch.int64, device="cuda")
    for params in (SamplingParams(temperature=0.5, top_k=50, top_p=0.9),
                   SamplingParams(temperature=1.0, top_k=1024, top_p=1.0),
                   SamplingParams(temperature=0.0)):
        _check_rows(x, params, u)
        _check_rows(x, params, u, forbidden=(3,), by_row=by_row)


def test_sample_all_equal_row_takes_the_lowest_ids():
    """Every id ties: greedy takes id 0 (or the first one not forbidden) and
    top-k sampling draws among ids 0..k-1."""
    rows, vocab = 4, 16384
    x = torch.zeros(rows, vocab, dtype=torch.bfloat16, device="cuda")
    tok, _ = Sampler(SamplingParams()).sample_with_logprobs(x)
    assert tok[:, 0].tolist() == [0] * rows
    tok, _ = Sampler(SamplingParams()).sample_with_logprobs(x, forbidden_token_ids=(0, 1))
    assert tok[:, 0].tolist() == [2] * rows
    u = torch.tensor([0.0, 0.3, 0.7, 0.999], device="cuda")
    tok, lp = Sampler(SamplingParams(temperature=1.0, top_k=8)).sample_with_logprobs(x, uniforms=u)
    assert tok[:, 0].tolist() == [0, 2, 5, 7]
    assert torch.allclose(lp[:, 0].cpu(), torch.full((rows,), -float(np.log(vocab))), atol=1e-5)


def test_sample_step_reads_device_step_and_forbid_window():
    rows, vocab = 8, 6400
    g = torch.Generator(device="cuda").manual_seed(9)
    x = (torch.randn(rows, vocab, generator=g, device="cuda") * 2).to(torch.bfloat16)
    x[:, 7] = 20.0  # dominant id, forbidden only inside the window
    table = stateless_uniforms(list(range(rows)), 6, torch.device("cuda"))
    ids = torch.tensor([7], dtype=torch.int32, device="cuda")
    p = SamplingParams(temperature=0.5, top_k=40, top_p=0.9)
    for s in (0, 1, 2, 5, 9):  # step 9 is clamped to the last column
        step = torch.tensor([s], dtype=torch.int64, device="cuda")
        tok, _ = sample_step(x, p, table, step, ids, forbid_before_step=2)
        col = min(s, 5)
        ref = Sampler(p).sample_with_logprobs(
            x, uniforms=table[:, col], forbidden_token_ids=(7,) if s < 2 else ())[0][:, 0]
        assert torch.equal(tok, ref), s
        assert bool((tok == 7).all()) == (s >= 2)


def test_sample_graph_replays_advance_the_step():
    rows, vocab = 8, 16384
    g = torch.Generator(device="cuda").manual_seed(4)
    x = (torch.randn(rows, vocab, generator=g, device="cuda") * 2).to(torch.bfloat16)
    table = stateless_uniforms([77 + r for r in range(rows)], 5, torch.device("cuda"))
    p = SamplingParams(temperature=0.35, top_k=50, top_p=0.9)
    step = torch.zeros(1, dtype=torch.int64, device="cuda")
    tok = torch.empty(rows, dtype=torch.int64, device="cuda")
    lp = torch.empty(rows, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        sample_step(x, p, table, step, out=(tok, lp))
        with torch.cuda.graph(graph, stream=s):
            sample_step(x, p, table, step, out=(tok, lp))
            step.add_(1)
    torch.cuda.current_stream().wait_stream(s)
    step.zero_()
    for t in range(5):
        graph.replay()
        torch.cuda.synchronize()
        ref = Sampler(p).sample_with_logprobs(x, uniforms=table[:, t])[0][:, 0]
        assert torch.equal(tok, ref), t


def test_sample_rejects_unsupported():
    x = torch.zeros(2, 64, dtype=torch.bfloat16, device="cuda")
    u = torch.full((2,), 0.5, device="cuda")
    with pytest.raises(ValueError, match="not built"):
        Sampler(SamplingParams(temperature=1.0, top_k=0, top_p=0.9)).sample_with_logprobs(
            x, uniforms=u)
    with pytest.raises(ValueError, match="not built"):
        Sampler(SamplingParams(temperature=1.0, top_k=2000)).sample_with_logprobs(x, uniforms=u)
    with pytest.raises(ValueError, match="outside the vocabulary"):
        Sampler(SamplingParams(temperature=1.0, top_k=5)).sample_with_logprobs(
            x, uniforms=u, forbidden_token_ids=(64,))
    with pytest.raises(ValueError, match="mutually exclusive"):
        Sampler(SamplingParams(temperature=1.0, top_k=5)).sample_with_logprobs(
            x, uniforms=u, generator=torch.Generator(device="cuda"))
    with pytest.raises(ValueError, match="uniforms must match"):
        Sampler(SamplingParams(temperature=1.0, top_k=5)).sample_with_logprobs(
            x, uniforms=torch.full((3,), 0.5, device="cuda"))
