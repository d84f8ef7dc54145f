"""Page-index metadata on the GPU vs the oracle: bit-exact.

Covers the integer part of the backend (python/aios/attention/flashinfer.py:
209-250 and get_last_indices :111-112): ``prepare_metadata``'s cu_seqlens,
flat page indices and last-token rows, the device gather behind it
(``aios_build_indices``), and the graph path's fixed-buffer metadata
(``Mi355xStaticDecodeMetadata.refresh``), against oracle/metadata.py with
exact equality.  Known answers: resources/lesson-26-flashinfer-backend/
run_lesson26.py:2-17 and resources/lesson-32-flashinfer-paged-attention/
run_lesson32.py:14-29 (requests in swapped page-table rows).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import metadata as omd

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def backend_ctx():
    """A backend with a global context holding a GPU page table and a KV
    pool (prepare_metadata reads both, as flashinfer.py:210-212 does)."""
    from aios_amd.attention import Mi355xAttentionBackend
    from aios_amd.config import ModelConfig
    from aios_amd.core import Context, reset_global_ctx, set_global_ctx
    from aios_amd.kvcache import MHAKVCache

    c = ModelConfig(num_layers=1, num_qo_heads=8, num_kv_heads=2, head_dim=96, hidden_size=768,
                    vocab_size=64, intermediate_size=128)
    backend = Mi355xAttentionBackend(c, workspace_size=16 << 20)
    reset_global_ctx()
    ctx = Context(page_size=1)
    ctx.kv_cache = MHAKVCache(2, 1, 96, 64, 1, torch.bfloat16, torch.device(DEV))
    ctx.attn_backend = backend
    set_global_ctx(ctx)
    yield backend, ctx
    reset_global_ctx()


def _batch(phase, q_lens, k_lens, rows, shared=0):
    from aios_amd.core import Batch, Req, SamplingParams

    reqs = [Req(input_ids=torch.empty(k, dtype=torch.long), cached_len=k - q, output_len=1,
                uid=i, sampling_params=SamplingParams(max_tokens=1), table_idx=r)
            for i, (q, k, r) in enumerate(zip(q_lens, k_lens, rows))]
    b = Batch(reqs=reqs, phase=phase)
    b.shared_prefix_len = shared
    return b


def _check(md, expect, bs):
    torch.cuda.synchronize()
    for name, got in (("cu_seqlens_q", md.cu_seqlens_q_gpu), ("cu_seqlens_k", md.cu_seqlens_k_gpu),
                      ("cu_seqlens_q", md.cu_seqlens_q_cpu), ("cu_seqlens_k", md.cu_seqlens_k_cpu),
                      ("indices", md.indices)):
        assert got.dtype == torch.int32, name
        np.testing.assert_array_equal(got.cpu().numpy(), expect[name], err_msg=name)
    last = md.get_last_indices(bs)
    assert last.dtype == torch.long
    np.testing.assert_array_equal(last.cpu().numpy(), expect["last_indices"])
    np.testing.assert_array_equal(md.last_page_len_cpu.numpy(), expect["last_page_len"])
    np.testing.assert_array_equal(md.seq_lens_cpu.numpy(), expect["seq_lens"])


def test_prepare_metadata_lesson26_known_answer(backend_ctx):
    backend, ctx = backend_ctx
    table = torch.full((2, 5), -1, dtype=torch.int32)
    table[0, :3] = torch.tensor([7, 4, 9])
    table[1, :5] = torch.tensor([2, 8, 1, 6, 3])
    ctx.page_table = table.to(DEV)
    batch = _batch("prefill", [3, 2], [3, 5], [0, 1])
    md = backend.prepare_metadata(batch)
    assert batch.attn_metadata is md
    expect = omd.build_metadata([3, 2], [3, 5], table.numpy(), [0, 1])
    # the literal answer of run_lesson26.py, independent of the oracle
    assert expect["indices"].tolist() == [7, 4, 9, 2, 8, 1, 6, 3]
    assert expect["last_indices"].tolist() == [2, 4]
    _check(md, expect, 2)


def test_prepare_metadata_lesson32_swapped_rows(backend_ctx):
    backend, ctx = backend_ctx
    table = torch.full((4, 5), -1, dtype=torch.int32)
    table[3, :3] = torch.tensor([10, 11, 12])
    table[1, :5] = torch.tensor([20, 21, 22, 23, 24])
    ctx.page_table = table.to(DEV)
    md = backend.prepare_metadata(_batch("prefill", [3, 2], [3, 5], [3, 1]))
    expect = omd.build_metadata([3, 2], [3, 5], table.numpy(), [3, 1])
    assert expect["indices"].tolist() == [10, 11, 12, 20, 21, 22, 23, 24]
    _check(md, expect, 2)


def test_prepare_metadata_long_context_decode_table(backend_ctx):
    """The long-context decode shape: 24 rows x (4096 shared + U{0..64} + 1)
    positions of a 4224-wide table over a 65,536-page pool, rows fed in a
    non-monotone order."""
    backend, ctx = backend_ctx
    g = torch.Generator().manual_seed(20260814)
    n, p, width = 24, 4096, 4224
    perm = torch.randperm(65536, generator=g).to(torch.int32)
    table = torch.full((n + 3, width), -1, dtype=torch.int32)
    rows = torch.randperm(n + 3, generator=g)[:n].tolist()
    lens = (p + torch.randint(0, 65, (n,), generator=g) + 1).tolist()
    nxt = p
    for r, ln in zip(rows, lens):
        table[r, :p] = perm[:p]
        table[r, p:ln] = perm[nxt:nxt + ln - p]
        nxt += ln - p
    ctx.page_table = table.to(DEV)
    md = backend.prepare_metadata(_batch("decode", [1] * n, lens, rows, shared=p))
    expect = omd.build_metadata([1] * n, lens, table.numpy(), rows)
    assert len(expect["indices"]) == sum(lens)
    _check(md, expect, n)
    assert md.plan.prefix_len == p and md.plan.num_prefix_chunks > 1  # the cascade plan


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_build_indices_ragged_rows(seed):
    """aios_build_indices on ragged rows (empty ones included), repeated and
    non-monotone row ids and a padded page-table stride."""
    from aios_amd import _lib

    g = torch.Generator().manual_seed(seed)
    n_rows, stride, width = 9, 1030, 1000
    table = torch.randint(0, 1 << 20, (n_rows, stride), generator=g, dtype=torch.int32)
    bs = 13
    row_ids = torch.randint(0, n_rows, (bs,), generator=g, dtype=torch.int32)
    lens = torch.randint(0, width + 1, (bs,), generator=g)
    lens[seed % bs] = 0
    lens[(seed + 5) % bs] = width
    cu_k = omd.cumulative(lens.tolist())
    total = int(cu_k[-1])
    # every device buffer the launch reads is held by a name until it has run
    table_d = table.to(DEV)
    rows_d = row_ids.to(DEV)
    cu_k_d = torch.from_numpy(cu_k).to(DEV)
    assert int(rows_d.max()) < n_rows and int(cu_k_d[-1]) == total
    out = torch.full((total,), -7, dtype=torch.int32, device=DEV)
    _lib.check(_lib.lib().aios_build_indices(
        table_d.data_ptr(), stride, rows_d.data_ptr(), cu_k_d.data_ptr(), bs, total,
        out.data_ptr(), torch.cuda.current_stream().cuda_stream), "aios_build_indices")
    torch.cuda.synchronize()
    del table_d, rows_d, cu_k_d
    expect = omd.build_metadata([1] * bs, lens.tolist(), table.numpy(), row_ids.tolist())
    np.testing.assert_array_equal(out.cpu().numpy(), expect["indices"])


def test_static_decode_refresh_matches_oracle(backend_ctx):
    """The graph path's metadata: one plan for the KV capacity, cu_seqlens_k
    and the indices rewritten on the device from a device kv_len."""
    backend, ctx = backend_ctx
    g = torch.Generator().manual_seed(3)
    n, cap, p = 8, 96, 40
    table = torch.randint(0, 64, (n, 128), generator=g, dtype=torch.int32)
    table[:, :p] = table[0, :p]
    table_d = table.to(DEV)
    ctx.page_table = table_d
    row_ids = torch.tensor([5, 0, 7, 2, 1, 6, 3, 4], dtype=torch.int32)
    md = backend.prepare_static_decode(row_ids.to(DEV), cap, p, table_d)
    for kv_len in (p + 1, p + 2, 63, cap):
        md.refresh(torch.tensor([kv_len], dtype=torch.int32, device=DEV))
        torch.cuda.synchronize()
        expect = omd.build_metadata([1] * n, [kv_len] * n, table.numpy(), row_ids.tolist())
        np.testing.assert_array_equal(md.cu_seqlens_k_gpu.cpu().numpy(), expect["cu_seqlens_k"])
        np.testing.assert_array_equal(md.indices[: n * kv_len].cpu().numpy(), expect["indices"])
        np.testing.assert_array_equal(md.get_last_indices(n).cpu().numpy(),
                                      expect["last_indices"])


def _decode_case(ctx, n=6, p=40, seed=11):
    """A CandidateGroup-shaped decode batch: n rows sharing p prefix pages,
    ragged suffixes, each row's new token on its last page."""
    from aios_amd.kvcache import MHAKVCache

    g = torch.Generator().manual_seed(seed)
    pool = 512
    ctx.kv_cache = MHAKVCache(2, 1, 96, pool, 1, torch.bfloat16, torch.device(DEV))
    ctx.kv_cache._kv_buffer.copy_(
        (torch.randn(ctx.kv_cache._kv_buffer.shape, generator=g) * 0.5).to(torch.bfloat16))
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    lens = (p + 1 + torch.randint(0, 9, (n,), generator=g)).tolist()
    table = torch.zeros((n, 64), dtype=torch.int32)
    nxt = p
    for r, ln in enumerate(lens):
        table[r, :p] = perm[:p]
        table[r, p:ln] = perm[nxt:nxt + ln - p]
        nxt += ln - p
    ctx.page_table = table.to(DEV)
    out_loc = torch.tensor([int(table[r, ln - 1]) for r, ln in enumerate(lens)],
                           dtype=torch.int32, device=DEV)
    q = (torch.randn(n, 8, 96, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    k = (torch.randn(n, 2, 96, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    v = (torch.randn(n, 2, 96, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    return lens, out_loc, q, k, v


def _run_decode(backend, ctx, lens, out_loc, q, k, v, p, fused):
    batch = _batch("decode", [1] * len(lens), lens, list(range(len(lens))), shared=p)
    batch.out_loc = out_loc
    batch.fused_append = fused
    backend.prepare_metadata(batch)
    out = backend.forward(q, k, v, ctx.kv_cache, 0, batch)
    torch.cuda.synchronize()
    return out


def test_fused_append_is_opt_in_and_equal(backend_ctx):
    """Without Batch.fused_append the backend runs store_kv then decode; with
    it, one launch: outputs and caches bit-equal."""
    backend, ctx = backend_ctx
    p = 40
    lens, out_loc, q, k, v = _decode_case(ctx, p=p)
    pool0 = ctx.kv_cache._kv_buffer.clone()
    plain = _run_decode(backend, ctx, lens, out_loc, q, k, v, p, fused=False)
    cache_plain = ctx.kv_cache._kv_buffer.clone()
    ctx.kv_cache._kv_buffer.copy_(pool0)
    backend.validate = True
    fused = _run_decode(backend, ctx, lens, out_loc, q, k, v, p, fused=True)
    assert torch.equal(plain, fused)
    assert torch.equal(cache_plain, ctx.kv_cache._kv_buffer)


def test_validation_rejects_broken_preconditions(backend_ctx):
    """validate=True: an out_loc that is not each row's last page, or a
    shared_prefix_len the rows do not share, raises before any launch."""
    backend, ctx = backend_ctx
    backend.validate = True
    p = 40
    lens, out_loc, q, k, v = _decode_case(ctx, p=p)
    pool0 = ctx.kv_cache._kv_buffer.clone()
    wrong = out_loc.clone()
    wrong[2] = out_loc[3]
    with pytest.raises(ValueError, match="last page"):
        _run_decode(backend, ctx, lens, wrong, q, k, v, p, fused=True)
    with pytest.raises(ValueError, match="share"):
        _run_decode(backend, ctx, lens, out_loc, q, k, v, p + 1, fused=False)
    assert torch.equal(pool0, ctx.kv_cache._kv_buffer)  # nothing was written
