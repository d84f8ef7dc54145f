"""Block-AttnRes depth mixer kernel (aios_attnres_mix / _ex) vs the float64
oracle (oracle/attnres.py) on the same bf16 inputs.

Tolerance: the mixer's output is bf16 and its weights are rounded to bf16
before the sum (kernel/attnres.py:92-97); a weight whose fp32 softmax sits
next to a bf16 rounding boundary may round the other way than in float64,
which moves the output by up to 2^-8 of that source.  The bound is the
path's 1e-2 tolerance (atol and rtol); the mean error is also checked to stay at
bf16 rounding level.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from aios_amd.kernel import attnres_mix, attnres_mix_step
from oracle import attnres as oar

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(torch.bfloat16)


def _inputs(s, n, d, with_partial, seed):
    bank = _bf16((s, n, d), seed)
    # sources of different scales, as deltas of different blocks have
    bank *= torch.linspace(0.5, 2.0, s, device=DEV).to(torch.bfloat16)[:, None, None]
    partial = _bf16((n, d), seed + 1, 1.5) if with_partial else None
    query = _bf16((d,), seed + 2, 0.2)
    knw = _bf16((d,), seed + 3).abs() + 0.5
    wq = (query.float() * knw.float()).contiguous()
    return bank, partial, query, knw, wq


def _np(t):
    return None if t is None else t.float().cpu().numpy()


def _check(out, want):
    got = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - want)
    assert np.all(err <= 1e-2 + 1e-2 * np.abs(want)), err.max()
    # bf16 output rounding is 2^-9 relative; the mean stays well under it
    assert err.mean() <= 4e-3 * max(1.0, np.abs(want).mean())


CASES = [
    (1, 8, 768, False),    # the first mixer of a forward: the embedding only
    (5, 8, 768, True),     # tests/test_ime_attnres.py:88-108 shape
    (9, 8, 768, False),    # the final mixer of the 8-block trunk
    (8, 64, 768, True),    # prefill of a 64-token prefix
    (3, 7, 1024, True),    # the one-wavefront-per-token kernel: hidden 256..1024
    (6, 9, 256, True),
    (12, 4, 1280, True),   # the workgroup kernel, all sources in registers
    (16, 5, 256, True),    # 17 sources: the re-reading path
    (40, 3, 8192, True),   # widest hidden, 41 sources
    (2, 1, 8, False),      # smallest hidden
]


@pytest.mark.parametrize("s,n,d,with_partial", CASES)
def test_attnres_mix_matches_oracle(s, n, d, with_partial):
    eps = 1e-6
    bank, partial, query, knw, wq = _inputs(s, n, d, with_partial, 100 + s + d)
    total = s + int(with_partial)
    scores = torch.full((total + 2, n), 123.0, device=DEV)
    out = attnres_mix(bank, partial, wq, eps, score_buffer=scores)
    torch.cuda.synchronize()
    want = oar.mix(_np(bank), _np(partial), _np(query), _np(knw), eps)
    _check(out, want)
    sc_want = oar.scores(_np(bank), _np(partial), _np(query), _np(knw), eps)
    sc_got = scores[:total].cpu().numpy()
    assert np.allclose(sc_got, sc_want, rtol=1e-4, atol=1e-4)
    assert bool((scores[total:] == 123.0).all())  # rows past the sources untouched


def test_attnres_zero_query_is_uniform_mean():
    """tests/test_ime_attnres.py:59-66 on the GPU (values exact in bf16)."""
    bank = torch.arange(3 * 2 * 8, dtype=torch.float32, device=DEV).reshape(3, 2, 8)
    bank = bank.to(torch.bfloat16)
    partial = torch.full((2, 8), 100.0, device=DEV, dtype=torch.bfloat16)
    out = attnres_mix(bank, partial, torch.zeros(8, device=DEV), 1e-6)
    want = torch.cat((bank, partial[None]), 0).float().mean(0)
    assert torch.equal(out.float(), want.to(torch.bfloat16).float())


@pytest.mark.parametrize("s,d", [(4, 768), (4, 1280), (20, 512)])
def test_attnres_step_fuses_partial_update(s, d):
    n = 8
    bank, partial, query, knw, wq = _inputs(s, n, d, True, 7)
    delta = _bf16((n, d), 9, 0.7)
    p_out = torch.empty_like(partial)
    out = attnres_mix_step(bank, partial, delta, wq, 1e-5, p_out)
    assert torch.equal(p_out, partial + delta)  # bf16 add, rounded once like torch's
    assert torch.equal(out, attnres_mix(bank, p_out, wq, 1e-5))
    # no partial: the delta is the partial
    out2 = attnres_mix_step(bank, None, delta, wq, 1e-5, p_out)
    assert torch.equal(p_out, delta)
    assert torch.equal(out2, attnres_mix(bank, delta, wq, 1e-5))
    # in place: partial_out is the partial itself
    p = partial.clone()
    out3 = attnres_mix_step(bank, p, delta, wq, 1e-5, p)
    assert torch.equal(p, partial + delta)
    assert torch.equal(out3, out)


def test_attnres_step_writes_next_bank_slot():
    """The block's last mix stores the new depth source into the bank's next
    slot; the result equals mixing the grown bank with no partial."""
    s, n, d = 3, 8, 768
    storage = torch.zeros((9, n, d), device=DEV, dtype=torch.bfloat16)
    storage[:s] = _bf16((s, n, d), 21)
    partial = _bf16((n, d), 22)
    delta = _bf16((n, d), 23, 0.5)
    wq = (_bf16((d,), 24, 0.2).float() * 1.1).contiguous()
    out = attnres_mix_step(storage[:s], partial, delta, wq, 1e-6, storage[s])
    assert torch.equal(storage[s], partial + delta)
    assert bool((storage[s + 1:] == 0).all())
    assert torch.equal(out, attnres_mix(storage[: s + 1], None, wq, 1e-6))


def test_attnres_graph_replays_match_eager():
    s, n, d = 6, 8, 768
    bank, partial, _, _, wq = _inputs(s, n, d, True, 31)
    delta = _bf16((n, d), 32)
    p_out = torch.empty_like(partial)
    out = torch.empty_like(partial)
    want = attnres_mix_step(bank, partial, delta, wq, 1e-6, torch.empty_like(partial))
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        attnres_mix_step(bank, partial, delta, wq, 1e-6, p_out, output_buffer=out)
        with torch.cuda.graph(graph, stream=stream):
            attnres_mix_step(bank, partial, delta, wq, 1e-6, p_out, output_buffer=out)
    torch.cuda.current_stream().wait_stream(stream)
    for i in range(3):
        out.zero_()
        p_out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
        assert torch.equal(p_out, partial + delta), i


def test_attnres_rejects_bad_shapes():
    bank = _bf16((2, 4, 768), 1)
    wq = torch.zeros(768, device=DEV)
    with pytest.raises(ValueError, match="partial must match bank"):
        attnres_mix(bank, _bf16((4, 512), 2), wq, 1e-6)
    with pytest.raises(ValueError, match="weighted_query must match hidden size"):
        attnres_mix(bank, None, torch.zeros(512, device=DEV), 1e-6)
    with pytest.raises(ValueError, match="bank must have shape"):
        attnres_mix(bank[0], None, wq, 1e-6)
    with pytest.raises(ValueError, match="multiple of 8"):
        attnres_mix(_bf16((2, 4, 100), 3), None, torch.zeros(100, device=DEV), 1e-6)
    with pytest.raises(ValueError, match="sources"):
        attnres_mix(_bf16((64, 2, 64), 4), _bf16((2, 64), 5), torch.zeros(64, device=DEV), 1e-6)
    with pytest.raises(ValueError, match="overlap"):
        storage = _bf16((3, 4, 768), 6)
        attnres_mix_step(storage[:2], None, _bf16((4, 768), 7), wq, 1e-6, storage[1])
