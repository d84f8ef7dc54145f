"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Each oracle function is checked against something other than its own
formula: the known answers the reference's resources hold (literal data
below, with the file they come from), an independent library routine
(numpy fancy-index assignment, torch's scaled_dot_product_attention), closed
forms, and invariants chosen so that a dropped term, a wrong sign, a wrong
head/page index or a transposed operand fails at least one of them.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from aios_amd.workloads import OP_TEST, make_decode_workload
from oracle import attention as oatt
from oracle import kv_store, metadata, prefix
from oracle.model import OracleModel, _rope, top3_by_average
from oracle.sdpa_cpu import paged_attention_cpu, sdpa_prefill_attention

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# --- paged KV scatter ---------------------------------------------------------

def test_scatter_known_answer_lesson30():
    """resources/lesson-30-triton-kv-store/run_lesson30.py:13-22: indices
    [17, 4, 9], width 8, token t row = t*100 + offset, 20 rows of -1."""
    width = 8
    values = np.array([[t * 100 + o for o in range(width)] for t in range(3)], dtype=np.int64)
    cache = np.full((20, width), -1, dtype=np.int64)
    out = kv_store.scatter_rows(cache, np.array([17, 4, 9]), values)
    assert out[17].tolist() == list(range(0, 8))
    assert out[4].tolist() == list(range(100, 108))
    assert out[9].tolist() == list(range(200, 208))
    untouched = [r for r in range(20) if r not in (17, 4, 9)]
    assert (out[untouched] == -1).all()
    assert (cache == -1).all()  # input not modified


def test_store_kv_matches_fancy_index_assignment():
    rng = np.random.default_rng(0)
    k_cache = rng.integers(0, 1 << 16, (64, 2, 96), dtype=np.uint16)
    v_cache = rng.integers(0, 1 << 16, (64, 2, 96), dtype=np.uint16)
    idx = rng.permutation(64)[:13].astype(np.int32)
    k = rng.integers(0, 1 << 16, (13, 2, 96), dtype=np.uint16)
    v = rng.integers(0, 1 << 16, (13, 2, 96), dtype=np.uint16)
    ko, vo = kv_store.store_kv(k_cache, v_cache, idx, k, v)
    ke, ve = k_cache.copy(), v_cache.copy()
    ke[idx] = k
    ve[idx] = v
    assert np.array_equal(ko, ke) and np.array_equal(vo, ve)
    assert not np.array_equal(ko, vo)  # K and V halves are not swapped


@pytest.mark.parametrize("bad", ["cache_ndim", "layout", "count"])
def test_store_kv_validation(bad):
    kc = np.zeros((8, 2, 4), np.uint16)
    k = np.zeros((3, 2, 4), np.uint16)
    idx = np.arange(3)
    if bad == "cache_ndim":
        kc = kc.reshape(8, 8)
    elif bad == "layout":
        k = np.zeros((3, 4, 2), np.uint16)
    else:
        idx = np.arange(2)
    with pytest.raises(ValueError):
        kv_store.store_kv(kc, kc if kc.ndim == 3 else kc, idx, k, k)


# --- metadata -----------------------------------------------------------------

def test_metadata_known_answer_lesson26():
    """resources/lesson-26-flashinfer-backend/run_lesson26.py:2-17."""
    pages = [[7, 4, 9], [2, 8, 1, 6, 3]]
    table = np.full((2, 5), -1, dtype=np.int32)
    for r, p in enumerate(pages):
        table[r, : len(p)] = p
    md = metadata.build_metadata([3, 2], [3, 5], table, [0, 1])
    assert md["cu_seqlens_q"].tolist() == [0, 3, 5]
    assert md["cu_seqlens_k"].tolist() == [0, 3, 8]
    assert md["indices"].tolist() == [7, 4, 9, 2, 8, 1, 6, 3]
    assert md["last_indices"].tolist() == [2, 4]
    assert md["last_page_len"].tolist() == [1, 1]


def test_metadata_known_answer_lesson32_row_order():
    """resources/lesson-32-flashinfer-paged-attention/run_lesson32.py:14-29,
    with the requests stored in swapped page-table rows."""
    table = np.full((4, 5), -1, dtype=np.int32)
    table[3, :3] = [10, 11, 12]
    table[1, :5] = [20, 21, 22, 23, 24]
    md = metadata.build_metadata([3, 2], [3, 5], table, [3, 1])
    assert md["cu_seqlens_q"].tolist() == [0, 3, 5]
    assert md["cu_seqlens_k"].tolist() == [0, 3, 8]
    assert md["indices"].tolist() == [10, 11, 12, 20, 21, 22, 23, 24]


# --- attention ----------------------------------------------------------------

def _offset_causal_sdpa(q, k, v, cached, scale):
    """torch's SDPA with an explicit boolean mask (independent of the oracle)."""
    g = q.shape[1] // k.shape[1]
    qb = torch.from_numpy(q).double().transpose(0, 1)
    kb = torch.from_numpy(k).double().transpose(0, 1).repeat_interleave(g, 0)
    vb = torch.from_numpy(v).double().transpose(0, 1).repeat_interleave(g, 0)
    qpos = torch.arange(cached, cached + q.shape[0])[:, None]
    kpos = torch.arange(k.shape[0])[None, :]
    out = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=kpos <= qpos, scale=scale)
    return out.transpose(0, 1).numpy()


@pytest.mark.parametrize("cached", [0, 2])
def test_reference_offset_causal_case_seed17(cached):
    """tests/test_attention_backend.py:25-53 (seed 17, q_len 3, 4q/2kv, D=8)
    against torch SDPA and the committed fixture."""
    fx = np.load(os.path.join(GOLDEN, "offset_causal.npz"))
    g = torch.Generator().manual_seed(17)
    q = torch.randn(3, 4, 8, generator=g).numpy()
    k = torch.randn(cached + 3, 2, 8, generator=g).numpy()
    v = torch.randn(cached + 3, 2, 8, generator=g).numpy()
    assert np.array_equal(q, fx[f"q{cached}"]) and np.array_equal(k, fx[f"k{cached}"])
    out = oatt.attention_one(q, k, v, cached, 8 ** -0.5)
    np.testing.assert_allclose(out, _offset_causal_sdpa(q, k, v, cached, 8 ** -0.5),
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out, fx[f"out{cached}"], rtol=0, atol=0)


@pytest.mark.parametrize("shape", [(5, 8, 2, 96, 7), (1, 4, 4, 64, 0), (9, 12, 4, 128, 30)])
def test_attention_matches_sdpa_random(shape):
    lq, hq, hkv, d, cached = shape
    rng = np.random.default_rng(lq * 1000 + d)
    q = rng.standard_normal((lq, hq, d))
    k = rng.standard_normal((cached + lq, hkv, d))
    v = rng.standard_normal((cached + lq, hkv, d))
    np.testing.assert_allclose(oatt.attention_one(q, k, v, cached, d ** -0.5),
                               _offset_causal_sdpa(q, k, v, cached, d ** -0.5),
                               rtol=1e-10, atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    lq, hq, hkv, d = 4, 8, 2, 16
    # Constant keys: uniform weights over the visible keys -> running means of v.
    q = rng.standard_normal((lq, hq, d))
    k = np.ones((lq, hkv, d))
    v = rng.standard_normal((lq, hkv, d))
    out = oatt.attention_one(q, k, v, 0, 0.25)
    for i in range(lq):
        means = v[: i + 1].mean(axis=0)  # [hkv, d]
        np.testing.assert_allclose(out[i], np.repeat(means, hq // hkv, axis=0), atol=1e-12)
    # First query with cached_len 0 sees only key 0 -> exactly v[0].
    np.testing.assert_allclose(out[0], np.repeat(v[0], hq // hkv, axis=0), atol=1e-15)
    # GQA mapping: query head h reads kv head h // G (not h % Hkv).
    vv = np.zeros((2, hkv, d))
    vv[:, 0] = 1.0
    vv[:, 1] = 2.0
    out = oatt.attention_one(rng.standard_normal((1, hq, d)), rng.standard_normal((2, hkv, d)),
                             vv, 1, 1.0)
    assert np.allclose(out[0, :4], 1.0) and np.allclose(out[0, 4:], 2.0)
    # Two keys, scores a and b: weights are the logistic of (a - b) * scale.
    qq = np.zeros((1, 1, 2))
    qq[0, 0] = [1.0, 0.0]
    kk = np.array([[[3.0, 0.0]], [[-1.0, 0.0]]])
    vk = np.array([[[1.0, 0.0]], [[0.0, 1.0]]])
    o = oatt.attention_one(qq, kk, vk, 1, 0.5)
    w0 = 1.0 / (1.0 + math.exp(-(3.0 - -1.0) * 0.5))
    np.testing.assert_allclose(o[0, 0], [w0, 1.0 - w0], atol=1e-15)


def test_paged_attention_page_permutation_and_decode():
    rng = np.random.default_rng(5)
    hq, hkv, d, pages = 8, 2, 32, 40
    kc = rng.standard_normal((pages, hkv, d))
    vc = rng.standard_normal((pages, hkv, d))
    kv_lens = [7, 1, 12]
    perm = rng.permutation(pages)
    idx = perm[: sum(kv_lens)].astype(np.int32)
    cu_k = metadata.cumulative(kv_lens)
    q = rng.standard_normal((3, hq, d))
    out = oatt.decode_attention(q, kc, vc, idx, cu_k, d ** -0.5)
    # relabel the physical pages: same logical KV -> same output
    relabel = rng.permutation(pages)
    kc2 = np.empty_like(kc)
    vc2 = np.empty_like(vc)
    kc2[relabel] = kc
    vc2[relabel] = vc
    out2 = oatt.decode_attention(q, kc2, vc2, relabel[idx].astype(np.int32), cu_k, d ** -0.5)
    np.testing.assert_allclose(out, out2, atol=1e-14)
    # decode row b == offset-causal attention with cached_len = kv_len - 1
    for b in range(3):
        pg = idx[cu_k[b]:cu_k[b + 1]]
        ref = _offset_causal_sdpa(q[b : b + 1], kc[pg], vc[pg], kv_lens[b] - 1, d ** -0.5)
        np.testing.assert_allclose(out[b : b + 1], ref, atol=1e-12)


def test_online_softmax_known_answer_lesson41():
    """resources/lesson-41-flashattention-online-softmax/run_lesson41.py:20-24:
    scores [1, 2, 5, -1], values [[1,0],[0,1],[2,2],[-1,3]], blocks 1/2/3."""
    scores = [1.0, 2.0, 5.0, -1.0]
    values = [[1, 0], [0, 1], [2, 2], [-1, 3]]
    e = [math.exp(s - 5.0) for s in scores]
    z = sum(e)
    naive = [sum(w * v[j] for w, v in zip(e, values)) / z for j in range(2)]
    for block in (1, 2, 3, 4):
        out, m, l = oatt.online_softmax(scores, values, block)
        np.testing.assert_allclose(out, naive, rtol=1e-14)
        assert m == 5.0
        np.testing.assert_allclose(l, z, rtol=1e-14)


def test_merge_states_split_anywhere_equals_unsplit():
    rng = np.random.default_rng(11)
    hq, hkv, d, n = 8, 2, 16, 23
    q = rng.standard_normal((hq, d))
    k = rng.standard_normal((n, hkv, d)) * 2.0
    v = rng.standard_normal((n, hkv, d))
    full = oatt.attention_one(q[None], k, v, n - 1, d ** -0.5)[0]
    o_all, lse_all = oatt.partial_state(q, k, v, d ** -0.5)
    np.testing.assert_allclose(o_all, full, atol=1e-13)
    for cuts in ([5], [1, 2, 20], [0, 23], [11, 11, 12]):
        bounds = [0, *cuts, n]
        parts = [oatt.partial_state(q, k[a:b], v[a:b], d ** -0.5)
                 for a, b in zip(bounds[:-1], bounds[1:])]
        o, lse = oatt.merge_states(parts)
        np.testing.assert_allclose(o, full, atol=1e-13)
        np.testing.assert_allclose(lse, lse_all, atol=1e-12)
    # an empty suffix leaves the prefix result unchanged
    empty = oatt.partial_state(q, k[:0], v[:0], d ** -0.5)
    assert np.isneginf(empty[1]).all()
    o, _ = oatt.merge_states([(o_all, lse_all), empty])
    np.testing.assert_allclose(o, o_all, atol=0)


def test_sdpa_cpu_restatement_matches_oracle():
    rng = np.random.default_rng(2)
    hq, hkv, d, pages = 8, 2, 96, 64
    kc = torch.from_numpy(rng.standard_normal((pages, hkv, d)))
    vc = torch.from_numpy(rng.standard_normal((pages, hkv, d)))
    q_lens, kv_lens = [3, 1, 5], [3, 9, 12]
    idx = torch.from_numpy(rng.permutation(pages)[: sum(kv_lens)].astype(np.int32))
    cu_q = metadata.cumulative(q_lens)
    cu_k = metadata.cumulative(kv_lens)
    q = torch.from_numpy(rng.standard_normal((sum(q_lens), hq, d)))
    got = paged_attention_cpu(q, kc, vc, idx, cu_q, cu_k, d ** -0.5)
    ref = oatt.paged_attention(q.numpy(), kc.numpy(), vc.numpy(), idx.numpy(), cu_q, cu_k,
                               d ** -0.5)
    np.testing.assert_allclose(got.numpy(), ref.reshape(sum(q_lens), -1), atol=1e-12)
    with pytest.raises(ValueError, match="cached_len"):
        sdpa_prefill_attention(q[:2], kc[:3], vc[:3], cached_len=2, sm_scale=1.0)


def test_op_test_golden_fixture():
    """The seeded op-test workload regenerates bit-identically and the oracle
    reproduces the committed output."""
    fx = np.load(os.path.join(GOLDEN, "op_test_decode.npz"))
    wl = make_decode_workload(OP_TEST, seed=int(fx["seed"]))
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits(wl.q[0]), fx["q_bits"])
    assert np.array_equal(bits(wl.k_cache[0]), fx["k_bits"])
    assert np.array_equal(bits(wl.v_cache[0]), fx["v_bits"])
    assert np.array_equal(wl.indices.numpy(), fx["indices"])
    assert np.array_equal(wl.cu_k.numpy(), fx["cu_k"])
    # every row shares the same 24 prefix pages
    cu = fx["cu_k"]
    pre = [fx["indices"][cu[b]: cu[b] + 24].tolist() for b in range(8)]
    assert all(p == pre[0] for p in pre)
    f64 = lambda t: t.to(torch.float64).numpy()
    out = oatt.decode_attention(f64(wl.q[0]), f64(wl.k_cache[0]), f64(wl.v_cache[0]),
                                wl.indices.numpy(), wl.cu_k.numpy(), 96 ** -0.5)
    np.testing.assert_allclose(out, fx["out"], rtol=0, atol=1e-15)


# --- prefix reuse ---------------------------------------------------------------

@pytest.mark.parametrize("case", [
    # resources/lesson-14-prefix-kv-reuse/run_lesson14.py:26-37 (old pages 10.., new 100..)
    ("same", [1, 2, 3], [1, 2, 3], (3, [10, 11, 12], [], [])),
    ("append", [1, 2, 3], [1, 2, 3, 4, 5], (3, [10, 11, 12], [], [100, 101])),
    ("retokenized tail", [1, 2, 3, 4], [1, 2, 8, 9], (2, [10, 11], [12, 13], [100, 101])),
    ("backspace", [1, 2, 3, 4], [1, 2, 3], (0, [], [10, 11, 12, 13], [100, 101, 102])),
], ids=lambda c: c[0] if isinstance(c, tuple) else None)
def test_prefix_plan_known_answers_lesson14(case):
    _, old, new, expect = case
    got = prefix.plan_prefix(old, list(range(10, 10 + len(old))), new)
    assert got[:4] == expect


def test_token_lcp():
    assert prefix.token_lcp([], [1]) == 0
    assert prefix.token_lcp([1, 2, 3], [1, 2]) == 2
    assert prefix.token_lcp([4], [5]) == 0


# --- model oracle building blocks ----------------------------------------------

def test_rope_closed_forms():
    rng = torch.Generator().manual_seed(0)
    x = torch.randn(1, 5, 2, 8, generator=rng)
    pos = torch.tensor([0, 1, 2, 7, 100])
    y = _rope(x, pos, 10000.0)
    assert torch.allclose(y[:, 0], x[:, 0])  # position 0 is the identity
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), atol=1e-5)  # rotation
    # pair (i, i + D/2) rotates by pos * theta^(-2i/D)
    for p_i, p in enumerate(pos.tolist()):
        for i in range(4):
            ang = p * 10000.0 ** (-2 * i / 8)
            a, b = x[0, p_i, 0, i].item(), x[0, p_i, 0, i + 4].item()
            assert abs(y[0, p_i, 0, i].item() - (a * math.cos(ang) - b * math.sin(ang))) < 1e-4
            assert abs(y[0, p_i, 0, i + 4].item() - (b * math.cos(ang) + a * math.sin(ang))) < 1e-4


def _tiny_config(**kw):
    from aios_amd.config import ModelConfig

    base = dict(num_layers=2, num_qo_heads=4, num_kv_heads=2, head_dim=16, hidden_size=32,
                vocab_size=50, intermediate_size=24, rms_norm_eps=1e-6)
    base.update(kw)
    return ModelConfig(**base)


def test_oracle_model_zero_blocks_is_normalised_embedding():
    """With every projection zero the decoder is the identity on the residual:
    logits = RMSNorm(embed[ids]) @ embed^T."""
    from aios_amd.qwen3 import init_weights

    c = _tiny_config()
    w = init_weights(c, 0, "cpu", dtype=torch.float32, std=0.1)
    for lw in w["layers"]:
        for key in ("qkv", "o", "gate_up", "down"):
            lw[key].zero_()
    ids = torch.tensor([[3, 7, 7, 1]])
    e = w["embed"][ids]
    ref = (e * torch.rsqrt(e.pow(2).mean(-1, keepdim=True) + c.rms_norm_eps)) @ w["embed"].T
    assert torch.allclose(OracleModel(c, w).logits(ids), ref, atol=1e-5)


class _DenseCpuBackend:
    """Test double for the attention backend: dense offset-causal attention on
    the CPU via the float64 oracle, no KV cache (one full-sequence prefill)."""

    def __init__(self, scale):
        self.scale = scale

    def prepare_metadata(self, batch):
        class _M:
            def get_last_indices(self, bs):
                return torch.tensor([batch.input_ids.numel() - 1])
        batch.attn_metadata = _M()

    def forward(self, q, k, v, kv_cache, layer_id, batch):
        out = oatt.attention_one(q.double().numpy(), k.double().numpy(), v.double().numpy(), 0,
                                 self.scale)
        return torch.from_numpy(out).to(q.dtype).reshape(q.shape[0], -1)


def test_oracle_model_matches_product_decoder_composition():
    """The oracle's plain pre-norm decoder and the product decoder's fused
    residual-add form (qwen3.py structure) agree in float32 on the CPU."""
    from aios_amd.core import Batch, Context, Req, SamplingParams, reset_global_ctx, set_global_ctx
    from aios_amd.qwen3 import Qwen3ForCausalLM, init_weights

    c = _tiny_config(num_layers=3)
    w = init_weights(c, 1, "cpu", dtype=torch.float32, std=0.2)
    g = torch.Generator().manual_seed(3)
    for lw in w["layers"]:  # non-trivial norm weights
        for key in ("input_norm", "post_norm", "q_norm", "k_norm"):
            lw[key].uniform_(0.5, 1.5, generator=g)
    ids = torch.tensor([5, 9, 2, 44, 0, 13])
    backend = _DenseCpuBackend(c.head_dim ** -0.5)
    from tests.util import TorchOps

    model = Qwen3ForCausalLM(c, w, "cpu", attn_backend=backend, max_positions=64, ops=TorchOps())
    reset_global_ctx()
    ctx = Context(page_size=1)
    ctx.kv_cache = None
    set_global_ctx(ctx)
    try:
        req = Req(input_ids=ids, cached_len=0, output_len=1, uid=0,
                  sampling_params=SamplingParams(), table_idx=0)
        batch = Batch(reqs=[req], phase="prefill", return_all_logits=True)
        batch.input_ids = ids
        batch.positions = torch.arange(len(ids), dtype=torch.int32)
        backend.prepare_metadata(batch)
        with ctx.forward_batch(batch):
            got = model.forward()
    finally:
        reset_global_ctx()
    ref = OracleModel(c, w).logits(ids[None])[0]
    assert torch.allclose(got, ref, atol=1e-4, rtol=1e-4)


def test_top3_by_average_distinct_and_ordered():
    ids = torch.tensor([[1, 2], [3, 4], [1, 2], [5, 6], [7, 8]])
    avg = torch.tensor([-1.0, -0.5, -0.2, -3.0, -0.9])
    assert top3_by_average(ids, avg) == [(1, 2), (3, 4), (7, 8)]


# --- Block-AttnRes depth mixer ------------------------------------------------

from oracle import attnres as oar  # noqa: E402


def test_round_bf16_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 10.0,
                        # exact ties between two bf16 values (round to even)
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8)],
                                 dtype=np.float32),
                        np.array([np.inf, -np.inf, 0.0, -0.0], dtype=np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(oar.round_bf16(x), want)


def test_attnres_zero_query_is_uniform_depth_mean():
    """Known answer of tests/test_ime_attnres.py:59-66: bank = arange(48)
    as [3, 2, 8], partial = 100, zero query -> mean of the four sources."""
    bank = np.arange(3 * 2 * 8, dtype=np.float64).reshape(3, 2, 8)
    partial = np.full((2, 8), 100.0)
    got = oar.mix(bank, partial, np.zeros(8), np.ones(8), 1e-6)
    want = (bank.sum(axis=0) + partial) / 4.0
    assert np.allclose(got, want, rtol=0, atol=1e-12)


def test_attnres_expanded_equals_materialized():
    """tests/test_ime_attnres.py:47-56: the direct (expanded) mixer equals the
    materialised reference; their query / key-norm weights, seed 7."""
    g = torch.Generator().manual_seed(7)
    bank = torch.randn(4, 5, 8, generator=g).double().numpy()
    partial = torch.randn(5, 8, generator=g).double().numpy()
    query = np.array([0.3, -0.2, 0.1, 0.4, -0.5, 0.6, 0.2, -0.1])
    knw = np.array([1.0, 0.9, 1.1, 0.8, 1.2, 1.0, 0.7, 1.3])
    for p in (None, partial):
        a = oar.mix(bank, p, query, knw, 1e-6, round_weights=False)
        b = oar.mix_materialized(bank, p, query, knw, 1e-6, round_weights=False)
        assert np.allclose(a, b, rtol=1e-12, atol=1e-12)
    # A dropped key-norm weight or eps, or a sum instead of a mean, changes it.
    base = oar.mix(bank, partial, query, knw, 1e-6, round_weights=False)
    assert not np.allclose(base, oar.mix(bank, partial, query, np.ones(8), 1e-6, False))
    assert not np.allclose(base, oar.mix(bank, partial, query, knw, 1.0, False))


def test_attnres_hand_computed_two_sources():
    """D = 4, x0 = [3, 4, 0, 0], x1 = [0, 0, 1, 1], query e0, key-norm
    weight [2, 1, 1, 1], eps 0: scores 3*2/2.5 = 2.4 and 0; softmax weights
    0.9168273 / 0.0831727, bf16 0.91796875 / 0.0830078125."""
    bank = np.array([[[3.0, 4.0, 0.0, 0.0]], [[0.0, 0.0, 1.0, 1.0]]])
    q = np.array([1.0, 0.0, 0.0, 0.0])
    knw = np.array([2.0, 1.0, 1.0, 1.0])
    sc = oar.scores(bank, None, q, knw, 0.0)
    assert np.allclose(sc[:, 0], [2.4, 0.0], atol=1e-12)
    w = oar.softmax_weights(sc)
    assert w[:, 0].tolist() == [0.91796875, 0.0830078125]
    got = oar.mix(bank, None, q, knw, 0.0)
    assert np.allclose(got[0], [2.75390625, 3.671875, 0.0830078125, 0.0830078125], atol=1e-12)
    # the partial as a last source is the same as a third bank source
    third = np.array([[0.5, -1.0, 2.0, 0.0]])
    a = oar.mix(bank, third, q, knw, 1e-6)
    b = oar.mix(np.concatenate([bank, third[None]]), None, q, knw, 1e-6)
    assert np.array_equal(a, b)


def test_attnres_closed_forms():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((1, 6, 32))
    q = rng.standard_normal(32)
    knw = rng.uniform(0.5, 1.5, 32)
    # one source: weight 1, output = the source
    assert np.allclose(oar.mix(x, None, q, knw, 1e-6), x[0], atol=0)
    # identical sources: output = that source (weights sum to 1 before rounding)
    same = np.repeat(x, 4, axis=0)
    assert np.allclose(oar.mix(same, None, q, knw, 1e-6, round_weights=False), x[0], atol=1e-12)
    # RMS normalisation: scaling a source leaves its score unchanged (eps = 0)
    bank = rng.standard_normal((3, 6, 32))
    s1 = oar.scores(bank, None, q, knw, 0.0)
    bank2 = bank.copy()
    bank2[1] *= 7.5
    s2 = oar.scores(bank2, None, q, knw, 0.0)
    assert np.allclose(s1, s2, rtol=1e-12, atol=1e-12)
    # a dominant score selects its source
    big = bank.copy()
    big[2] = np.sign(q * knw)[None, :] * 5.0
    out = oar.mix(big, None, q * 100.0, knw, 1e-6, round_weights=False)
    assert np.allclose(out, big[2], atol=1e-6)


def _tiny_attnres(**kw):
    base = dict(num_layers=8, residual_type="block_attnres", attnres_num_blocks=2)
    base.update(kw)
    return _tiny_config(**base)


def test_attnres_config_gates():
    """tests/test_ime_attnres.py:81-85: partial migration and a bad layer
    partition are rejected."""
    with pytest.raises(ValueError, match="alpha=1.0"):
        _tiny_attnres(attnres_alpha=0.5)
    with pytest.raises(ValueError, match="divisible"):
        _tiny_attnres(num_layers=7)
    assert _tiny_attnres().layers_per_attnres_block == 4


def test_oracle_attnres_zero_blocks_is_normalised_embedding():
    """Zero projections and zero routing queries: every delta is zero, every
    mixer averages its sources, the final mixer returns embed / 3 (bank of
    the embedding and two zero blocks) and the final RMSNorm removes the
    scale: logits = RMSNorm(embed[ids]) @ embed^T."""
    from aios_amd.qwen3 import init_weights

    c = _tiny_attnres(rms_norm_eps=1e-12)
    w = init_weights(c, 0, "cpu", dtype=torch.float32, std=0.1)
    for lw in w["layers"]:
        for key in ("qkv", "o", "gate_up", "down", "attn_res_query", "mlp_res_query"):
            lw[key].zero_()
    w["final_res_query"].zero_()
    ids = torch.tensor([[3, 7, 7, 1]])
    e = w["embed"][ids]
    ref = (e * torch.rsqrt(e.pow(2).mean(-1, keepdim=True))) @ w["embed"].T
    assert torch.allclose(OracleModel(c, w).logits(ids), ref, atol=1e-5)


def test_oracle_attnres_model_matches_product_composition():
    """The oracle's list-of-sources trunk with materialised mixers and the
    product's fused form (expanded mixers, partial formed inside the next
    mixer, block sums written into the bank's next slot) agree in float32."""
    from aios_amd.core import Batch, Context, Req, SamplingParams, reset_global_ctx, set_global_ctx
    from aios_amd.minimind_ime import MiniMindBlockAttnResForCausalLM
    from aios_amd.qwen3 import init_weights
    from tests.util import TorchOps

    c = _tiny_attnres()
    w = init_weights(c, 2, "cpu", dtype=torch.float32, std=0.2)
    g = torch.Generator().manual_seed(3)
    for lw in w["layers"]:
        for key in ("input_norm", "post_norm", "q_norm", "k_norm", "attn_res_norm",
                    "mlp_res_norm"):
            lw[key].uniform_(0.5, 1.5, generator=g)
        lw["attn_res_query"].mul_(20.0)  # routing far from uniform
        lw["mlp_res_query"].mul_(20.0)
    w["final_res_query"].mul_(20.0)
    ids = torch.tensor([5, 9, 2, 44, 0, 13, 8])
    backend = _DenseCpuBackend(c.head_dim ** -0.5)
    model = MiniMindBlockAttnResForCausalLM(c, w, "cpu", attn_backend=backend, max_positions=64,
                                            ops=TorchOps())
    reset_global_ctx()
    ctx = Context(page_size=1)
    ctx.kv_cache = None
    set_global_ctx(ctx)
    try:
        req = Req(input_ids=ids, cached_len=0, output_len=1, uid=0,
                  sampling_params=SamplingParams(), table_idx=0)
        batch = Batch(reqs=[req], phase="prefill", return_all_logits=True)
        batch.input_ids = ids
        batch.positions = torch.arange(len(ids), dtype=torch.int32)
        backend.prepare_metadata(batch)
        with ctx.forward_batch(batch):
            got = model.forward()
    finally:
        reset_global_ctx()
    om = OracleModel(c, w)
    ref = om.logits(ids[None])[0]
    assert torch.allclose(got, ref, atol=1e-4, rtol=1e-4)
    # the mixers matter: the standard trunk on the same weights differs
    std = OracleModel(_tiny_config(num_layers=8), w).logits(ids[None])[0]
    assert not torch.allclose(std, ref, atol=1e-2)


# --- stateless candidate sampling --------------------------------------------

from oracle import sampling as osamp  # noqa: E402


def test_splitmix64_published_vector():
    """SplitMix64 (Vigna) with seed 1234567: the first five outputs of the
    published reference stream; step t of the reference's uniform is the
    generator's (t + 1)-th output (sample.py:12-21)."""
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert [osamp.splitmix64(1234567, t) for t in range(5)] == want


def test_stateless_uniforms_range_and_keying():
    u = osamp.stateless_uniforms([20260814 + i for i in range(8)], 12)
    assert u.shape == (8, 12) and u.dtype == np.float32
    assert (u > 0).all() and (u < 1).all()
    # keyed by (seed, step), not by row position: candidate 3's stream is the
    # same wherever it sits in the batch
    assert np.array_equal(osamp.stateless_uniforms([20260817], 12)[0], u[3])
    assert abs(float(u.mean()) - 0.5) < 0.1
    with pytest.raises(ValueError):
        osamp.stateless_uniforms([1], 0)


def test_sample_greedy_is_argmax_with_forbidden():
    x = np.array([0.1, 3.0, 3.0, -1.0, 2.5])
    tok, lp, _ = osamp.sample_row(x, 0.0, 0, 1.0, 0.5)
    assert tok == 1  # first index of the maximum
    assert np.isclose(lp, x[1] - np.log(np.exp(x).sum()))
    tok, lp, _ = osamp.sample_row(x, 0.7, 1, 1.0, 0.5, forbidden=[1, 2])
    assert tok == 4
    assert np.isclose(lp, x[4] - np.log(np.exp(x).sum()))  # raw, unmodified distribution


def test_sample_full_vocab_is_inverse_cdf():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(50) * 2
    t = 0.8
    p = np.exp(x / t - (x / t).max())
    p /= p.sum()
    cum = np.cumsum(p)
    for u in rng.uniform(0, 1, 200):
        tok, _, _ = osamp.sample_row(x, t, 0, 1.0, u)
        assert tok == min(int(np.searchsorted(cum, u, side="left")), len(x) - 1)


def test_sample_top_p_known_answer():
    """probs [0.5, 0.3, 0.15, 0.05], top_p 0.7: cumulative [0.5, 0.8, ...]
    removes ids 2 and 3 (the cumulative before them exceeds 0.7); the kept
    pair renormalises to [0.625, 0.375]."""
    x = np.log(np.array([0.5, 0.3, 0.15, 0.05]))
    assert osamp.sample_row(x, 1.0, 0, 0.7, 0.6)[0] == 0
    assert osamp.sample_row(x, 1.0, 0, 0.7, 0.63)[0] == 1
    assert osamp.sample_row(x, 1.0, 0, 0.7, 0.99)[0] == 1
    assert osamp.sample_row(x, 1.0, 4, 0.7, 0.99)[0] == 1  # same with top_k covering all


def test_sample_frequencies_match_truncated_distribution():
    """top_k 3 of 6 at temperature 0.5: over a fine u grid each candidate is
    drawn with its renormalised probability; the others never."""
    x = np.array([1.0, -0.5, 2.0, 0.3, 1.9, -2.0])
    s = x / 0.5
    top = np.argsort(-s)[:3]
    p = np.exp(s[top] - s[top].max())
    p /= p.sum()
    grid = (np.arange(20000) + 0.5) / 20000
    counts = {}
    for u in grid:
        tok = osamp.sample_row(x, 0.5, 3, 1.0, u)[0]
        counts[tok] = counts.get(tok, 0) + 1
    assert set(counts) == set(top.tolist())
    for i, t in enumerate(top):
        assert abs(counts[int(t)] / len(grid) - p[i]) < 1e-3


def test_sample_ties_take_lower_id_first():
    x = np.array([0.0, 5.0, 1.0, 5.0, 5.0])
    # three-way tie at the top: top_k 2 keeps ids 1 and 3, in that order
    assert osamp.sample_row(x, 1.0, 2, 1.0, 0.25)[0] == 1
    assert osamp.sample_row(x, 1.0, 2, 1.0, 0.75)[0] == 3


from dataclasses import replace  # noqa: E402

from aios_amd.config import ModelConfig  # noqa: E402
from oracle.cpu_decoder import PagedCpuDecoder  # noqa: E402


def _small_cfg(**kw):
    base = dict(num_layers=2, num_qo_heads=4, num_kv_heads=2, head_dim=16, hidden_size=64,
                vocab_size=97, intermediate_size=96, rope_theta=10000.0)
    base.update(kw)
    return ModelConfig(**base)


def test_cpu_decoder_matches_dense_oracle():
    """The KV-cached CPU decoder (the full-model CPU baseline) in float32:
    prefix prefill, an LCP extension and three rows of decode steps over
    scattered pages give the dense oracle's last-position logits; relabelling
    the pages changes nothing (bitwise)."""
    from aios_amd.qwen3 import init_weights

    c = _small_cfg()
    w = init_weights(c, 5, "cpu", std=0.15)
    om = OracleModel(c, w)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(c.vocab_size, (9,), generator=g).tolist()
    conts = torch.randint(c.vocab_size, (3, 3), generator=g)

    def run(perm):
        dec = PagedCpuDecoder(c, w, torch.float32, num_pages=64)
        pages = perm[:9]
        first = dec.prefill(ids[:6], pages)
        ext = dec.prefill(ids, pages, cached_len=6)
        rows = [pages.clone() for _ in range(3)]
        nxt = 9
        steps = []
        for s in range(3):
            new = perm[nxt: nxt + 3]
            nxt += 3
            rows = [torch.cat([r, new[i: i + 1]]) for i, r in enumerate(rows)]
            steps.append(dec.decode(conts[:, s], rows, new))
        return first, ext, steps

    perm_a = torch.randperm(64, generator=g).to(torch.int32)
    perm_b = torch.randperm(64, generator=g).to(torch.int32)
    first, ext, steps = run(perm_a)
    ref = om.logits(torch.tensor([ids]), 0)[0]
    assert (first - ref[5]).abs().max() < 1e-4
    assert (ext - ref[8]).abs().max() < 1e-4
    for s in range(3):
        seq = torch.cat([torch.tensor(ids).expand(3, -1), conts[:, : s + 1]], 1)
        want = om.logits(seq, seq.shape[1] - 1)[:, -1]
        assert (steps[s] - want).abs().max() < 1e-4, s
    first_b, ext_b, steps_b = run(perm_b)
    assert torch.equal(first, first_b) and torch.equal(ext, ext_b)
    assert all(torch.equal(x, y) for x, y in zip(steps, steps_b))


def test_cpu_decoder_bf16_close_to_fp32():
    from aios_amd.qwen3 import init_weights

    c = _small_cfg(head_dim=32, num_qo_heads=4, num_kv_heads=1, hidden_size=128)
    w = init_weights(c, 6, "cpu", std=0.1)
    ids = list(range(3, 20))
    pages = torch.randperm(32, generator=torch.Generator().manual_seed(6)).to(torch.int32)
    a = PagedCpuDecoder(c, w, torch.float32, num_pages=32).prefill(ids, pages)
    b = PagedCpuDecoder(c, w, torch.bfloat16, num_pages=32).prefill(ids, pages)
    assert (a - b).abs().max() < 0.1 * a.abs().max()
    with pytest.raises(ValueError, match="standard residual"):
        PagedCpuDecoder(replace(c, residual_type="block_attnres", attnres_num_blocks=1), w)
