"""aios_cg_step_prepare (the captured CandidateGroup step's page column,
decode metadata, step column and embedding rows in one launch) against the
same quantities built with torch from its definition; integer results and
copied rows bit-exact."""
from __future__ import annotations

import pytest
import torch

from aios_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(rows, pt_cols, max_kv_len, pos0, step, page_rows, hidden, vocab, seed, embed=True):
    g = torch.Generator().manual_seed(seed)
    pt = torch.randint(0, 1 << 20, (rows, pt_cols), generator=g, dtype=torch.int32)
    pages = torch.randint(0, 1 << 20, (page_rows, rows), generator=g, dtype=torch.int32)
    pos = torch.full((rows,), pos0, dtype=torch.int32)
    tokens = torch.randint(-3, vocab + 3, (rows,), generator=g, dtype=torch.long)
    table = torch.randn(vocab, hidden, generator=g).to(torch.bfloat16)
    d = {k: v.to(DEV) for k, v in dict(pt=pt, pages=pages, pos=pos, tokens=tokens,
                                        table=table).items()}
    stepv = torch.tensor([step], dtype=torch.long, device=DEV)
    step_next = torch.zeros(1, dtype=torch.long, device=DEV)
    out_loc = torch.zeros(rows, dtype=torch.int32, device=DEV)
    cu_k = torch.full((rows + 1,), -7, dtype=torch.int32, device=DEV)
    indices = torch.full((rows * max_kv_len,), -7, dtype=torch.int32, device=DEV)
    h = torch.zeros(rows, hidden, dtype=torch.bfloat16, device=DEV)
    lib = _lib.lib()
    _lib.check(lib.aios_cg_step_prepare(
        stepv.data_ptr(), d["pages"].data_ptr(), page_rows, rows, out_loc.data_ptr(),
        d["pt"].data_ptr(), d["pt"].stride(0), pt_cols, d["pos"].data_ptr(), cu_k.data_ptr(),
        indices.data_ptr(), max_kv_len, step_next.data_ptr(), d["tokens"].data_ptr(),
        d["table"].data_ptr() if embed else None, vocab, hidden,
        h.data_ptr() if embed else None, torch.cuda.current_stream().cuda_stream),
        "aios_cg_step_prepare")
    torch.cuda.synchronize()

    s = min(max(step, 0), page_rows - 1)
    loc = pages[s]
    pt_ref = pt.clone()
    if 0 <= pos0 < pt_cols:
        pt_ref[:, pos0] = loc
    L = min(max(pos0 + 1, 0), max_kv_len)
    assert torch.equal(out_loc.cpu(), loc)
    assert torch.equal(d["pt"].cpu(), pt_ref)
    assert torch.equal(cu_k.cpu(), torch.arange(rows + 1, dtype=torch.int32) * L)
    flat = indices.cpu()
    assert torch.equal(flat[: rows * L], pt_ref[:, :L].reshape(-1))
    assert bool((flat[rows * L:] == -7).all())  # nothing past rows * L written
    assert int(step_next.item()) == step + 1
    if embed:
        assert torch.equal(h.cpu(), table[tokens.clamp(0, vocab - 1)])
    else:
        assert not bool(h.any())


@pytest.mark.parametrize("rows,pos0,step", [(8, 37, 3), (24, 150, 11), (1, 0, 0), (5, 63, 0)])
def test_prepare_matches_definition(rows, pos0, step):
    _case(rows, 256, 200, pos0, step, page_rows=16, hidden=768, vocab=300, seed=rows + pos0)


def test_prepare_clamps_step_and_length_and_ids():
    # step past the pre-allocated pages -> the last row; pos + 1 past
    # max_kv_len -> max_kv_len; ids outside the table -> clamped
    _case(6, 128, 64, 99, 40, page_rows=4, hidden=64, vocab=50, seed=3)
    # a position past the page-table row writes no column
    _case(3, 32, 32, 40, 1, page_rows=4, hidden=8, vocab=10, seed=4)


def test_prepare_without_embedding():
    _case(8, 256, 128, 20, 2, page_rows=8, hidden=1024, vocab=64, seed=5, embed=False)
