"""Full-model parity: the CandidateGroup engine on the gfx950 backend vs the
float32 CPU oracle model (oracle/model.py) with the same seeded bf16 weights.

Acceptance follows the reference's backend equivalence check
(scripts/check_attnres_runtime_equivalence.py:37-47, 82-89, 234-251):
full-vocabulary logit max-abs within LOGIT_TOL, Top-1 / Top-3 token-id sets
of the logits equal (topk overlap at k in {1, 3}), identical discrete
decisions, and average log-probs within AVG_LP_TOL.  Synthetic N(0, 0.02)
weights give nearly flat next-token distributions (top-1/top-2 log-prob gaps
of a few 1e-3 occur in every 16-step run), while bf16 GPU logits differ from
float32 ones by about 0.03; so set equality is asserted wherever the oracle's
own margin exceeds SET_MARGIN = 2 * LOGIT_TOL_TIGHT (below that, either order is
a valid bf16 outcome), and every discrete GPU decision must be the oracle's
choice up to a gap of 2 * (observed logit deviation at that step).
"""
from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from aios_amd.config import MINIMIND_0P1B, MINIMIND_ATTNRES_0P214B, MINIMIND_IME_0P1B, QWEN3_0P6B
from aios_amd.core import reset_global_ctx
from aios_amd.ime import CancellationToken, CandidateGroupConfig, CandidateGroupEngine, CandidateGroupRuntime
from aios_amd.qwen3 import init_weights, weights_to
from oracle.model import OracleModel, top3_by_average

pytestmark = pytest.mark.gpu

LOGIT_TOL = 0.125        # reference equivalence-check default (bf16 full-vocab logits)
LOGIT_TOL_TIGHT = 0.05   # what this build holds itself to (measured ~0.03)
SET_MARGIN = 2 * LOGIT_TOL_TIGHT
AVG_LP_TOL = 0.02
# Seeds whose prefix logits have top-1 and top-3 margins above SET_MARGIN
# in the oracle (MiniMind-0.1B shape, 32-token prefix).
SCREENED_SEEDS = (4, 15, 22)


def _prefix(seed: int, n: int, vocab: int) -> list[int]:
    g = torch.Generator().manual_seed(seed)
    return torch.randint(vocab, (n,), generator=g).tolist()


def _engine(config, seed, num_pages=1024, use_graphs=False):
    """Eager engines by default: their decode steps can be observed one by one."""
    w = init_weights(config, seed, "cpu")
    rt = CandidateGroupRuntime(config, weights_to(w, "cuda"), "cuda", num_pages=num_pages)
    return CandidateGroupEngine(rt, use_graphs=use_graphs), OracleModel(config, w)


def _record_decode_logits(eng):
    """Wrap the decode step to keep each step's logits and active rows."""
    steps = []
    inner = eng._decode_step

    def wrapped(tokens, page_table, cached_len, rows, prefix_len):
        logits, pages = inner(tokens, page_table, cached_len, rows, prefix_len)
        steps.append((list(rows), logits.float().cpu()))
        return logits, pages

    eng._decode_step = wrapped
    return steps


def _set_equal_if_screened(gpu: torch.Tensor, ref: torch.Tensor, k: int) -> bool | None:
    """Top-k id sets must match when the oracle's k-th/k+1-th gap clears SET_MARGIN."""
    s = ref.sort(descending=True).values
    if (s[k - 1] - s[k]).item() <= SET_MARGIN:
        return None
    return set(gpu.topk(k).indices.tolist()) == set(ref.topk(k).indices.tolist())


def teardown_function(_):
    reset_global_ctx()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("seed", SCREENED_SEEDS)
def test_prefix_logits_and_top_sets(seed):
    c = MINIMIND_0P1B
    eng, om = _engine(c, seed)
    prefix = _prefix(seed, 32, c.vocab_size)
    res = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=1))
    gpu = res.prefix_logits[0].float().cpu()
    ref = om.logits(torch.tensor(prefix)[None], 31)[0, -1]
    diff = (gpu - ref).abs().max().item()
    assert diff <= LOGIT_TOL_TIGHT <= LOGIT_TOL, diff
    assert torch.nn.functional.cosine_similarity(gpu, ref, dim=0).item() > 0.999
    assert _set_equal_if_screened(gpu, ref, 1) is True
    assert _set_equal_if_screened(gpu, ref, 3) is True


@pytest.mark.parametrize("config", [MINIMIND_IME_0P1B.with_layers(4),
                                    replace(QWEN3_0P6B, num_layers=4, vocab_size=8192)],
                         ids=["minimind-ime-h64-g3", "qwen3-0.6b-h128-g2"])
def test_prefix_logits_other_shapes(config):
    eng, om = _engine(config, 3)
    prefix = _prefix(3, 48, config.vocab_size)
    res = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=1))
    gpu = res.prefix_logits[0].float().cpu()
    ref = om.logits(torch.tensor(prefix)[None], 47)[0, -1]
    assert (gpu - ref).abs().max().item() <= LOGIT_TOL_TIGHT


def _check_candidate_group(eng, om, prefix, n, steps):
    rec = _record_decode_logits(eng)
    res = eng.complete(prefix, CandidateGroupConfig(num_candidates=n, max_new_tokens=steps))
    assert not res.cancelled and len(res.raw_candidates) == n
    ids = torch.tensor([c.token_ids for c in res.raw_candidates])
    assert ids.shape == (n, steps)
    tf = om.teacher_forced(prefix, ids)  # oracle log-probs on the GPU's own histories
    # step 0: candidate i takes the i-th best first token
    ref0 = tf[0, 0]
    top_vals = ref0.sort(descending=True).values[:n]
    d0 = (res.prefix_logits[0].float().cpu().log_softmax(-1) - ref0).abs().max().item()
    assert d0 <= LOGIT_TOL_TIGHT
    chosen0 = ref0[ids[:, 0]]
    assert (chosen0 - top_vals).abs().max().item() <= 2 * d0 + 1e-6
    assert len(rec) == steps - 1
    checked_sets = 0
    for j, (rows, logits) in enumerate(rec, start=1):
        assert rows == list(range(n))
        ref = tf[:, j]
        gpu_lp = logits.log_softmax(-1)
        dev = (gpu_lp - ref).abs().max().item()
        assert dev <= LOGIT_TOL_TIGHT, (j, dev)
        tok = ids[:, j]
        assert torch.equal(tok, gpu_lp.argmax(-1))  # greedy on the GPU's logits
        gap = ref.max(-1).values - ref.gather(1, tok[:, None]).squeeze(1)
        assert gap.max().item() <= 2 * dev + 1e-6, (j, gap)
        for r in range(n):
            for k in (1, 3):
                ok = _set_equal_if_screened(logits[r], ref[r], k)
                if ok is not None:
                    assert ok, (j, r, k)
                    checked_sets += 1
    assert checked_sets >= n * (steps - 1) // 2  # most positions are screened in
    avg_ref = tf.gather(2, ids[:, :, None]).squeeze(2).mean(1)
    avg_gpu = torch.tensor([c.average_logprob for c in res.raw_candidates])
    assert (avg_ref - avg_gpu).abs().max().item() <= AVG_LP_TOL
    # Top-3 by average log-prob: the oracle's ranking of the same sequences
    # agrees wherever neighbouring averages are apart by more than AVG_LP_TOL.
    top_gpu = top3_by_average(ids, avg_gpu)
    assert [c.token_ids for c in res.candidates] == top_gpu
    order = torch.argsort(avg_ref, descending=True)
    a = avg_ref[order]
    if (a[2] - a[3]).item() > 2 * AVG_LP_TOL:
        assert set(top3_by_average(ids, avg_ref)) == set(top_gpu)
    if (a[0] - a[1]).item() > 2 * AVG_LP_TOL:
        assert top3_by_average(ids, avg_ref)[0] == top_gpu[0]
    return res


def test_candidate_group_h64_norm_rope_in_decode():
    """Head size 64 (the MiniMind-IME 0.1B shape, 4 layers): the decode steps
    take the q/k norm + rotation inside the decode launch; every eager step's
    logits against the oracle, then graph-replayed groups token for token
    equal to the eager ones."""
    c = MINIMIND_IME_0P1B.with_layers(4)
    eng, om = _engine(c, 11)
    be = eng.rt.model.attn_backend
    assert c.head_dim in be.ROPE_IN_DECODE_HEAD_DIMS
    calls = []
    inner = be.forward_rope

    def counted(*args, **kw):
        calls.append(1)
        return inner(*args, **kw)

    be.forward_rope = counted
    prefix = _prefix(11, 20, c.vocab_size)
    _check_candidate_group(eng, om, prefix, 8, 10)
    assert len(calls) == c.num_layers * 9  # every decode step after the first token
    eng.reset_prefix_cache()
    graphed = CandidateGroupEngine(eng.rt, use_graphs=True)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=10)
    for _ in range(2):
        e = eng.complete(prefix, cfg)
        eng.reset_prefix_cache()
        torch.cuda.synchronize()
        g = graphed.complete(prefix, cfg)
        graphed.reset_prefix_cache()
        assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in e.raw_candidates]
        assert [x.average_logprob for x in g.raw_candidates] == \
            [x.average_logprob for x in e.raw_candidates]


def test_candidate_group_minimind_0p1b():
    """Prefill a 32-token prefix, 8 candidates x 16 greedy steps over shared prefix KV."""
    c = MINIMIND_0P1B
    eng, om = _engine(c, 20260814)
    _check_candidate_group(eng, om, _prefix(20260814, 32, c.vocab_size), 8, 16)
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 32
    eng.reset_prefix_cache()
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages


def test_candidate_group_long_prefix_cascade():
    """Prefix >= 256 tokens: the decode plan uses the shared-prefix cascade."""
    c = replace(QWEN3_0P6B, num_layers=3, vocab_size=8192)
    eng, om = _engine(c, 11)
    prefix = _prefix(11, 300, c.vocab_size)
    plans = []
    inner = eng.rt.model.attn_backend.prepare_metadata

    def spy(batch):
        md = inner(batch)
        plans.append((batch.phase, md.plan.num_prefix_chunks, md.plan.prefix_len))
        return md

    eng.rt.model.attn_backend.prepare_metadata = spy
    _check_candidate_group(eng, om, prefix, 8, 6)
    decode_plans = [p for p in plans if p[0] == "decode"]
    assert decode_plans and all(p[2] == 300 and p[1] >= 1 for p in decode_plans)


def test_lcp_extension_and_strict_backspace():
    """Cross-keystroke reuse: +2 tokens prefills only the extension against the
    cached prefix; deleting back to the old prefix re-prefills from scratch."""
    c = replace(QWEN3_0P6B, num_layers=4, vocab_size=8192)
    eng, om = _engine(c, 5)
    base = _prefix(5, 128, c.vocab_size)
    ext = base + _prefix(6, 2, c.vocab_size)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=4)
    r0 = eng.complete(base, cfg)
    assert r0.reused_prefix_tokens == 0
    r1 = eng.complete(ext, cfg)
    assert r1.reused_prefix_tokens == 128 and r1.active_model_tokens == 2 + 8 * 3
    ref = om.logits(torch.tensor(ext)[None], 129)[0, -1]
    assert (r1.prefix_logits[0].float().cpu() - ref).abs().max().item() <= LOGIT_TOL_TIGHT
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 130
    r2 = eng.complete(base, cfg)  # strict backspace
    assert r2.reused_prefix_tokens == 0
    ref = om.logits(torch.tensor(base)[None], 127)[0, -1]
    assert (r2.prefix_logits[0].float().cpu() - ref).abs().max().item() <= LOGIT_TOL_TIGHT
    r3 = eng.complete(base, cfg)  # identical prefix: cached logits, no prefill
    assert r3.reused_prefix_tokens == 128 and r3.active_model_tokens == 8 * 3
    assert torch.equal(r3.prefix_logits, r2.prefix_logits)
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 128


def test_qwen3_0p6b_full_size_extension_and_decode():
    """The Qwen3-0.6B shape at full size (28 layers, 16q/8kv heads of 128,
    vocab 151,936): a 128-token prefix, its 2-token LCP extension prefilled
    against the cached prefix KV, then 8 candidates x 3 eager decode steps
    over the shared 130-token prefix (the cascade).  The extension's
    last-position logits, the first-token ranking, and two candidates' every
    decode step against the float32 oracle."""
    c = QWEN3_0P6B
    eng, om = _engine(c, 3)
    base = _prefix(3, 128, c.vocab_size)
    ext = base + _prefix(4, 2, c.vocab_size)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=3)
    eng.complete(base, cfg)
    rec = _record_decode_logits(eng)
    res = eng.complete(ext, cfg)
    assert res.reused_prefix_tokens == 128 and res.active_model_tokens == 2 + 8 * 2
    ref0 = om.logits(torch.tensor(ext)[None], 129)[0, -1].log_softmax(-1)
    gpu0 = res.prefix_logits[0].float().cpu().log_softmax(-1)
    d0 = (gpu0 - ref0).abs().max().item()
    assert d0 <= LOGIT_TOL_TIGHT, d0
    ids = torch.tensor([x.token_ids for x in res.raw_candidates])
    assert ids.shape == (8, 3)
    # candidate i starts from the GPU's i-th best first token; under the
    # oracle each is within 2 * d0 of the oracle's i-th best
    top_vals = ref0.sort(descending=True).values[:8]
    assert (ref0[ids[:, 0]] - top_vals).abs().max().item() <= 2 * d0 + 1e-6
    assert len(rec) == 2
    for r in (0, 5):
        seq = torch.tensor(ext + ids[r, :2].tolist())
        ref_r = om.logits(seq[None], len(ext))[0].log_softmax(-1)  # next-token at 130, 131
        for j, (rows, logits) in enumerate(rec):
            lp = logits[rows.index(r)].log_softmax(-1)
            dev = (lp - ref_r[j]).abs().max().item()
            assert dev <= LOGIT_TOL_TIGHT, (r, j, dev)
            tok = ids[r, j + 1]
            assert tok.item() == lp.argmax().item()
            assert (ref_r[j].max() - ref_r[j][tok]).item() <= 2 * dev + 1e-6, (r, j)
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 130


def test_cancelled_and_budget():
    c = MINIMIND_0P1B.with_layers(2)
    eng, _ = _engine(c, 1, num_pages=256)
    tok = CancellationToken(1)
    tok.cancel()
    res = eng.complete(_prefix(1, 32, c.vocab_size), CandidateGroupConfig(), cancellation=tok)
    assert res.cancelled and res.candidates == ()
    assert eng.rt.cache_manager.available_size == 256
    with pytest.raises(ValueError, match="KV budget"):
        eng.complete(_prefix(1, 200, c.vocab_size), CandidateGroupConfig(max_new_tokens=16))
    # a newer generation cancels the older one (latest wins)
    t1 = eng.new_generation()
    t2 = eng.new_generation()
    assert t1.cancelled and not t2.cancelled


def test_eos_compaction():
    """Rows whose token is EOS stop; the rest keep decoding as a compacted batch."""
    c = MINIMIND_0P1B.with_layers(4)
    eng, om = _engine(c, 9)
    prefix = _prefix(9, 32, c.vocab_size)
    first = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=6))
    ids = [cand.token_ids for cand in first.raw_candidates]
    eos = ids[2][0]  # candidate 2's first token becomes EOS
    rec = _record_decode_logits(eng)
    res = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=6,
                                                    eos_token_id=eos))
    assert res.raw_candidates[2].token_ids == () and res.raw_candidates[2].stop_reason == "eos"
    assert all(2 not in rows for rows, _ in rec)
    for i, cand in enumerate(res.raw_candidates):
        if i == 2 or not cand.token_ids:
            continue
        seq = torch.tensor([cand.token_ids])
        tf = om.teacher_forced(prefix, seq)[0]
        gap = tf.max(-1).values - tf.gather(1, seq[0][:, None]).squeeze(1)
        assert gap[1:].max().item() <= 2 * LOGIT_TOL_TIGHT
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 32


def _check_against_oracle(res, om, prefix, n, steps):
    """Oracle checks that need only the outputs (graph-replayed steps)."""
    ids = torch.tensor([c.token_ids for c in res.raw_candidates])
    assert ids.shape == (n, steps)
    tf = om.teacher_forced(prefix, ids)
    chosen = tf.gather(2, ids[:, :, None]).squeeze(2)
    top_vals = tf[0, 0].sort(descending=True).values[:n]
    assert (chosen[:, 0] - top_vals).abs().max().item() <= 2 * LOGIT_TOL_TIGHT
    gap = tf[:, 1:].max(-1).values - chosen[:, 1:]
    assert gap.max().item() <= 2 * LOGIT_TOL_TIGHT
    avg_gpu = torch.tensor([c.average_logprob for c in res.raw_candidates])
    assert (chosen.mean(1) - avg_gpu).abs().max().item() <= AVG_LP_TOL


def test_graph_replay_matches_eager_minimind_0p1b():
    """Graph-replayed decode steps give the eager loop's tokens and scores,
    on the first capture and on replays in later calls, with eager work and
    synchronisations between them."""
    c = MINIMIND_0P1B
    w = init_weights(c, 20260814, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=1024)
    eager = CandidateGroupEngine(rt, use_graphs=False)
    graphed = CandidateGroupEngine(rt, use_graphs=True)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=16)
    om = OracleModel(c, w)
    for seed in (20260814, 7, 20260814, 8):
        prefix = _prefix(seed, 32, c.vocab_size)
        e = eager.complete(prefix, cfg)
        eager.reset_prefix_cache()
        torch.cuda.synchronize()
        g = graphed.complete(prefix, cfg)
        graphed.reset_prefix_cache()
        assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in e.raw_candidates]
        assert [x.average_logprob for x in g.raw_candidates] == \
            [x.average_logprob for x in e.raw_candidates]
        assert g.active_model_tokens == e.active_model_tokens == 32 + 8 * 15
        _check_against_oracle(g, om, prefix, 8, 16)
    assert len(graphed._graphs) == 1
    assert rt.cache_manager.available_size == rt.num_pages


def test_graph_prefill_matches_eager():
    """Graph-replayed prefills and LCP extensions (up to 64 new tokens) give
    the eager prefill's logits and K/V rows bit for bit: on first use (the
    capture), on replays with eager work in between, for extensions of a
    cached prefix, and past the limit (eager in both engines).  The two
    engines share one runtime (one global context); each case's prefix K/V
    rows are copied out before the other engine runs it."""
    c = MINIMIND_0P1B.with_layers(3)
    w = init_weights(c, 12, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=512)
    graphed = CandidateGroupEngine(rt, use_graphs=True)
    eager = CandidateGroupEngine(rt, use_graphs=False)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=2)
    # (prefix, extension): the last two are the keystroke case over a longer
    # cached prefix (KV capacity 192 and 256, device-side kv_len and indices
    # built over the longer row)
    cases = [(5, 0), (9, 2), (9, 0), (31, 1), (5, 0), (40, 0), (70, 0), (9, 2), (128, 2),
             (250, 1)]
    for trial, (n, ext) in enumerate(cases):
        ids = _prefix(100 + trial, n + ext, c.vocab_size)
        res, kv = [], []
        for eng in (graphed, eager):
            if ext:
                eng.complete(ids[:n], cfg)
            r = eng.complete(ids, cfg)
            assert r.reused_prefix_tokens == (n if ext else 0)
            pages = eng._prefix_pages.long()
            kv.append((pages.clone(), [getattr(rt.kv_cache, kind)(layer)[pages].clone()
                                       for layer in range(c.num_layers)
                                       for kind in ("k_cache", "v_cache")]))
            res.append(r)
            eng.reset_prefix_cache()
            torch.cuda.synchronize()
        assert torch.equal(res[0].prefix_logits, res[1].prefix_logits), (n, ext)
        assert [x.token_ids for x in res[0].raw_candidates] == \
            [x.token_ids for x in res[1].raw_candidates]
        # the allocator hands out different pages the second time; their rows agree
        assert len(kv[0][0]) == len(kv[1][0]) == n + ext
        assert all(torch.equal(a, b) for a, b in zip(kv[0][1], kv[1][1])), (n, ext)
    assert sorted(graphed._prefill_graphs) == [(1, 64), (1, 256), (2, 64), (2, 192), (5, 64),
                                               (9, 64), (31, 64), (40, 64)]
    assert not eager._prefill_graphs
    assert rt.cache_manager.available_size == rt.num_pages


def test_graph_replay_cascade_prefix_and_neighbouring_lengths():
    """Long prefixes: the graph plans the cascade on a 64-aligned prefix and
    serves neighbouring prefix lengths from one capture.  The prefixes
    (320-350 tokens, planned prefix 320) lie above the planner's cascade
    threshold, and the captured plan is checked to hold a cascade, so the
    graph-replayed shared-prefix path (static metadata with prefix chunks,
    the prefix partials and the combine, indices built on the device) stays
    covered whatever the threshold."""
    c = replace(QWEN3_0P6B, num_layers=3, vocab_size=8192)
    eng, om = _engine(c, 12, use_graphs=True)
    for plen in (320, 321, 350):
        prefix = _prefix(plen, plen, c.vocab_size)
        res = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=6))
        _check_against_oracle(res, om, prefix, 8, 6)
        eng.reset_prefix_cache()
    assert len(eng._graphs) == 1
    plan = next(iter(eng._graphs.values())).md.plan
    assert plan.prefix_len == 320, plan.prefix_len
    assert plan.num_prefix_chunks >= 1, plan.num_prefix_chunks


def test_graph_replay_eos_masks_rows():
    c = MINIMIND_0P1B.with_layers(4)
    eng, om = _engine(c, 9, use_graphs=True)
    prefix = _prefix(9, 32, c.vocab_size)
    first = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=6))
    eos = first.raw_candidates[2].token_ids[0]
    res = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=6,
                                                    eos_token_id=eos))
    assert res.raw_candidates[2].token_ids == () and res.raw_candidates[2].stop_reason == "eos"
    for i, cand in enumerate(res.raw_candidates):
        assert eos not in cand.token_ids
        if i == 2 or not cand.token_ids:
            continue
        seq = torch.tensor([cand.token_ids])
        tf = om.teacher_forced(prefix, seq)[0]
        gap = tf.max(-1).values - tf.gather(1, seq[0][:, None]).squeeze(1)
        assert gap[1:].max().item() <= 2 * LOGIT_TOL_TIGHT
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 32



# --- Block-AttnRes (0.214B-shaped) trunk -----------------------------------------

def test_prefix_logits_attnres_0p214b():
    """64-token prefix through the 32-layer, 8-block depth-routed trunk (65
    mixers) vs the float32 oracle trunk."""
    c = MINIMIND_ATTNRES_0P214B
    eng, om = _engine(c, 3)
    prefix = _prefix(3, 64, c.vocab_size)
    res = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=1))
    gpu = res.prefix_logits[0].float().cpu()
    ref = om.logits(torch.tensor(prefix)[None], 63)[0, -1]
    assert (gpu - ref).abs().max().item() <= LOGIT_TOL_TIGHT
    assert torch.nn.functional.cosine_similarity(gpu, ref, dim=0).item() > 0.999
    for k in (1, 3):
        assert _set_equal_if_screened(gpu, ref, k) in (True, None)


def test_candidate_group_attnres_0p214b():
    """8 candidates x 12 greedy steps on the Block-AttnRes trunk: every
    decode step's logits against the oracle on the GPU's own histories."""
    c = MINIMIND_ATTNRES_0P214B
    eng, om = _engine(c, 20260814)
    _check_candidate_group(eng, om, _prefix(20260814, 64, c.vocab_size), 8, 12)
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages - 64


def test_graph_replay_matches_eager_attnres():
    c = MINIMIND_ATTNRES_0P214B.with_layers(8)
    w = init_weights(c, 5, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=1024)
    eager = CandidateGroupEngine(rt, use_graphs=False)
    graphed = CandidateGroupEngine(rt, use_graphs=True)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=10)
    om = OracleModel(c, w)
    for seed in (5, 6, 5):
        prefix = _prefix(seed, 64, c.vocab_size)
        e = eager.complete(prefix, cfg)
        eager.reset_prefix_cache()
        torch.cuda.synchronize()
        g = graphed.complete(prefix, cfg)
        graphed.reset_prefix_cache()
        assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in e.raw_candidates]
        assert [x.average_logprob for x in g.raw_candidates] == \
            [x.average_logprob for x in e.raw_candidates]
        _check_against_oracle(g, om, prefix, 8, 10)
    assert rt.cache_manager.available_size == rt.num_pages


# --- sampled candidates (the reference's default candidate rule) ------------

from aios_amd.core import SamplingParams  # noqa: E402
from oracle import sampling as osamp  # noqa: E402


def _check_sampled(res, prefix_logits, rec, cfg, n):
    """Every token of every candidate is what the sampling oracle draws from
    the GPU's own logits of that step with the candidate's stateless uniform
    (boundary cases: within 1e-5 of a cumulative sum, either neighbour)."""
    sp = cfg.sampling
    uni = osamp.stateless_uniforms([cfg.seed + i for i in range(n)], cfg.max_new_tokens)
    blocked = list(cfg.blocked_ids())
    steps = [(list(range(n)), prefix_logits.float().cpu().expand(n, -1))] + \
        [(rows, lg) for rows, lg in rec]
    checked = 0
    for j, (rows, lg) in enumerate(steps):
        for local, cand in enumerate(rows):
            tok = res.raw_candidates[cand].token_ids[j]
            fb = blocked if j < cfg.min_new_tokens else []
            want, _, d = osamp.sample_row(lg[local].numpy(), sp.temperature, sp.top_k, sp.top_p,
                                          float(uni[cand, j]), fb, detail=True)
            assert tok not in fb
            if d["u_margin"] > 1e-5 and d["cut_margin"] > 1e-5:
                assert tok == want, (j, cand, tok, want)
                checked += 1
            else:
                assert tok in set(d["order"].tolist())
    assert checked >= 0.9 * n * cfg.max_new_tokens


def test_candidate_group_sampled_minimind_0p1b():
    """The reference's first-round rule (temperature 0.35, top_k 50, top_p
    0.9, stateless uniforms keyed by seed + candidate), eager steps."""
    c = MINIMIND_0P1B
    eng, om = _engine(c, 20260814)
    prefix = _prefix(20260814, 32, c.vocab_size)
    rec = _record_decode_logits(eng)
    first = eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=1))
    top2 = first.prefix_logits[0].float().topk(2).indices.tolist()
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=12,
                               sampling=SamplingParams(temperature=0.35, top_k=50, top_p=0.9),
                               min_new_tokens=2, blocked_token_ids=tuple(top2))
    rec.clear()
    res = eng.complete(prefix, cfg)
    assert len(res.raw_candidates) == 8
    assert all(len(cand.token_ids) == 12 for cand in res.raw_candidates)
    _check_sampled(res, res.prefix_logits, rec, cfg, 8)
    # the two most likely first tokens are blocked for the first two steps
    assert all(cand.token_ids[0] not in top2 for cand in res.raw_candidates)
    # raw scores are the unmodified distribution's log-probs (oracle model)
    ids = torch.tensor([cand.token_ids for cand in res.raw_candidates])
    tf = om.teacher_forced(prefix, ids)
    avg_ref = tf.gather(2, ids[:, :, None]).squeeze(2).mean(1)
    avg_gpu = torch.tensor([cand.average_logprob for cand in res.raw_candidates])
    assert (avg_ref - avg_gpu).abs().max().item() <= AVG_LP_TOL


def test_graph_replay_matches_eager_sampled():
    c = MINIMIND_0P1B.with_layers(4)
    w = init_weights(c, 8, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=1024)
    eager = CandidateGroupEngine(rt, use_graphs=False)
    graphed = CandidateGroupEngine(rt, use_graphs=True)
    for seed in (1, 2, 1):
        cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=10, seed=100 + seed,
                                   sampling=SamplingParams(temperature=0.75, top_k=96, top_p=0.95),
                                   min_new_tokens=2, blocked_token_ids=(3, 4))
        prefix = _prefix(seed, 32, c.vocab_size)
        e = eager.complete(prefix, cfg)
        eager.reset_prefix_cache()
        torch.cuda.synchronize()
        g = graphed.complete(prefix, cfg)
        graphed.reset_prefix_cache()
        assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in e.raw_candidates]
        assert [x.average_logprob for x in g.raw_candidates] == \
            [x.average_logprob for x in e.raw_candidates]
    assert len(graphed._graphs) == 1


def test_runtime_from_exported_bundle(tmp_path):
    """A bundle written in the exporter's layout runs the same CandidateGroup
    as the in-memory weights it was written from (Block-AttnRes trunk)."""
    from aios_amd.weights import save_bundle

    c = MINIMIND_ATTNRES_0P214B.with_layers(8)
    w = init_weights(c, 12, "cpu")
    save_bundle(c, w, tmp_path)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=6)
    prefix = _prefix(12, 64, c.vocab_size)
    a = CandidateGroupEngine(CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda",
                                                   num_pages=512)).complete(prefix, cfg)
    reset_global_ctx()
    b = CandidateGroupEngine(CandidateGroupRuntime.from_bundle(tmp_path, "cuda",
                                                               num_pages=512)).complete(prefix, cfg)
    assert [x.token_ids for x in a.raw_candidates] == [x.token_ids for x in b.raw_candidates]
    assert [x.average_logprob for x in a.raw_candidates] == \
        [x.average_logprob for x in b.raw_candidates]


def test_candidate_group_adaptive_refill():
    """Refill rounds (ime.py:478-600, 333-370).  A greedy first round
    (top_k 1) yields one distinct candidate, so one refill round of 8
    branches follows at the refill schedule (temperature 0.75, top_k 96,
    top_p 0.95, seeds seed + 8 * 100003 + i) with the first round's
    sequence banned from step 2 on; every refill token is the sampling
    oracle's draw from the GPU's logits with that row's ban applied."""
    c = MINIMIND_0P1B.with_layers(4)
    eng, _ = _engine(c, 31)
    prefix = _prefix(31, 24, c.vocab_size)
    rec = _record_decode_logits(eng)
    t = 8
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=t, min_new_tokens=2,
                               sampling=SamplingParams(temperature=0.35, top_k=1, top_p=1.0),
                               max_candidates=24)
    res = eng.complete(prefix, cfg)
    raw = res.raw_candidates
    assert res.refill_rounds >= 1 and len(raw) == 8 + 8 * res.refill_rounds
    greedy = raw[0].token_ids
    assert all(r.token_ids == greedy for r in raw[:8]) and len(greedy) == t
    # round 2 against the oracle, with the ban
    sp = SamplingParams(temperature=0.75, top_k=96, top_p=0.95)
    uni = osamp.stateless_uniforms([cfg.seed + 8 * 100_003 + i for i in range(8)], t)
    steps = [(list(range(8)), res.prefix_logits.float().cpu().expand(8, -1))] + rec[t - 1: 2 * (t - 1)]
    checked = 0
    for j, (rows, lg) in enumerate(steps):
        assert rows == list(range(8))
        for r in rows:
            hist = raw[8 + r].token_ids
            fb = [greedy[j]] if j >= 2 and hist[:j] == greedy[:j] else []
            want, _, d = osamp.sample_row(lg[r].numpy(), sp.temperature, sp.top_k, sp.top_p,
                                          float(uni[r, j]), fb, detail=True)
            assert hist[j] not in fb
            if d["u_margin"] > 1e-5 and d["cut_margin"] > 1e-5:
                assert hist[j] == want, (j, r, hist[j], want)
                checked += 1
            else:
                assert hist[j] in set(d["order"].tolist())
    assert checked >= 0.9 * 8 * t
    assert all(r.token_ids != greedy for r in raw[8:16])
    shown = [x.token_ids for x in res.candidates]
    assert len(shown) == 3 and len(set(shown)) == 3
    eng.reset_prefix_cache()
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages
    # deterministic: the same request reproduces every round
    eng._decode_step = eng.__class__._decode_step.__get__(eng)
    again = eng.complete(prefix, cfg)
    assert [x.token_ids for x in again.raw_candidates] == [x.token_ids for x in raw]


def _record_rounds(eng):
    """Wrap the round generator: per round, (branches, sampling params, free
    pages on entry, pages the round allocated, banned sequences)."""
    rounds = []
    for name in ("_generate", "_generate_graphed"):
        inner = getattr(eng, name)

        def wrapped(prefix_logits, page_table, prefix_len, config, cancellation, banned=(),
                    _inner=inner):
            free = eng.rt.cache_manager.available_size
            out = _inner(prefix_logits, page_table, prefix_len, config, cancellation,
                         banned=banned)
            rounds.append((config.num_candidates, config.sampling, free,
                           sum(len(a) for a in out[1]), [tuple(b) for b in banned]))
            return out

        setattr(eng, name, wrapped)
    return rounds


def test_attnres_0p214b_refill_rounds():
    """The refill leg of the 0.214B Block-AttnRes model (full 32 layers): a greedy
    first round (top_k 1) leaves one distinct candidate, so sampled refill
    rounds of 8 x 32 steps follow up to 24 candidates (ime.py:478-600).
    Every round starts with only the prefix pages held (the previous round's
    suffix KV was freed, :588-592) and allocates 8 x 31 suffix pages; the
    rounds follow the refill schedule (temperature 0.75 + 0.10 r, top_k 96 +
    32 r); round 2's tokens are the sampling oracle's draws from the GPU's
    logits with the first round's sequence banned; graph-replayed rounds give
    the eager rounds' candidates; the prefix pages are all that remain."""
    c = MINIMIND_ATTNRES_0P214B
    eng, _ = _engine(c, 214)
    prefix = _prefix(214, 64, c.vocab_size)
    rec = _record_decode_logits(eng)
    rounds = _record_rounds(eng)
    t = 32
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=t, min_new_tokens=2,
                               sampling=SamplingParams(temperature=0.35, top_k=1, top_p=1.0),
                               max_candidates=24)
    res = eng.complete(prefix, cfg)
    raw = res.raw_candidates
    total = eng.rt.num_pages
    assert res.refill_rounds >= 1 and len(rounds) == 1 + res.refill_rounds
    assert len(raw) == sum(r[0] for r in rounds) <= 24
    for i, (n, sp, free, alloc, banned) in enumerate(rounds):
        assert free == total - len(prefix), (i, free)
        assert alloc == n * (t - 1), (i, alloc)
        if i:
            assert n == 8
            assert sp.temperature == pytest.approx(min(0.95, 0.75 + 0.10 * (i - 1)))
            assert sp.top_k == min(160, 96 + 32 * (i - 1)) and sp.top_p == 0.95
            assert banned, "every refill round bans the earlier candidates"
    assert eng.rt.cache_manager.available_size == total - len(prefix)
    greedy = raw[0].token_ids
    assert all(r.token_ids == greedy for r in raw[:8]) and len(greedy) == t
    sp = rounds[1][1]
    uni = osamp.stateless_uniforms([cfg.seed + 8 * 100_003 + i for i in range(8)], t)
    steps = [(list(range(8)), res.prefix_logits.float().cpu().expand(8, -1))] + rec[t - 1: 2 * (t - 1)]
    checked = 0
    for j, (rows, lg) in enumerate(steps):
        assert rows == list(range(8))
        for r in rows:
            hist = raw[8 + r].token_ids
            fb = [greedy[j]] if j >= 2 and hist[:j] == greedy[:j] else []
            want, _, d = osamp.sample_row(lg[r].numpy(), sp.temperature, sp.top_k, sp.top_p,
                                          float(uni[r, j]), fb, detail=True)
            assert hist[j] not in fb
            if d["u_margin"] > 1e-5 and d["cut_margin"] > 1e-5:
                assert hist[j] == want, (j, r, hist[j], want)
                checked += 1
            else:
                assert hist[j] in set(d["order"].tolist())
    assert checked >= 0.9 * 8 * t
    shown = [x.token_ids for x in res.candidates]
    assert len(shown) == 3 and len(set(shown)) == 3
    # graph-replayed rounds on the same runtime: the same candidates
    eng.reset_prefix_cache()
    graphed = CandidateGroupEngine(eng.rt, use_graphs=True)
    g_rounds = _record_rounds(graphed)
    g = graphed.complete(prefix, cfg)
    assert g.refill_rounds == res.refill_rounds
    assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in raw]
    assert [(r[0], r[2], r[3]) for r in g_rounds] == [(r[0], r[2], r[3]) for r in rounds]
    assert g.replayed_steps == sum(r[0] > 0 for r in g_rounds) * (t - 1)
    graphed.reset_prefix_cache()
    assert eng.rt.cache_manager.available_size == total


def test_graph_replay_matches_eager_refill():
    """Refill rounds replayed from captured graphs, with the banned-repeat
    rule evaluated on the device, give the eager rounds' candidates."""
    c = MINIMIND_0P1B.with_layers(4)
    w = init_weights(c, 8, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=1024)
    eager = CandidateGroupEngine(rt, use_graphs=False)
    graphed = CandidateGroupEngine(rt, use_graphs=True)
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=8, min_new_tokens=2,
                               sampling=SamplingParams(temperature=0.35, top_k=1, top_p=1.0),
                               max_candidates=24)
    for seed in (1, 2, 1):
        prefix = _prefix(seed, 32, c.vocab_size)
        e = eager.complete(prefix, cfg)
        eager.reset_prefix_cache()
        torch.cuda.synchronize()
        g = graphed.complete(prefix, cfg)
        graphed.reset_prefix_cache()
        assert e.refill_rounds >= 1 and g.refill_rounds == e.refill_rounds
        assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in e.raw_candidates]
        assert [x.average_logprob for x in g.raw_candidates] == \
            [x.average_logprob for x in e.raw_candidates]
        greedy = g.raw_candidates[0].token_ids
        assert all(x.token_ids != greedy for x in g.raw_candidates[8:])
    assert rt.cache_manager.available_size == rt.num_pages


def test_refill_budget_and_deadline():
    """The attempt budget caps a refill round (8 + 2 of max 10), and a
    deadline already passed when the first round ends stops refill
    (ime.py:511-517)."""
    c = MINIMIND_0P1B.with_layers(2)
    w = init_weights(c, 5, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=512)
    eng = CandidateGroupEngine(rt, use_graphs=True)
    base = dict(num_candidates=8, max_new_tokens=6, min_new_tokens=2,
                sampling=SamplingParams(temperature=0.35, top_k=1, top_p=1.0))
    prefix = _prefix(3, 16, c.vocab_size)
    r = eng.complete(prefix, CandidateGroupConfig(max_candidates=10, **base))
    eng.reset_prefix_cache()
    assert r.refill_rounds == 1 and len(r.raw_candidates) == 10
    r = eng.complete(prefix, CandidateGroupConfig(max_candidates=24, refill_deadline_ms=1e-6,
                                                  **base))
    eng.reset_prefix_cache()
    assert r.refill_rounds == 0 and len(r.raw_candidates) == 8
    # one distinct valid candidate: the display set holds it once
    assert [x.token_ids for x in r.candidates] == [r.raw_candidates[0].token_ids]
    assert rt.cache_manager.available_size == rt.num_pages


def test_graph_refill_pad_fill_matches_eager():
    """With the tokenizer's pad id as the ban-table fill (ime.py:990-996),
    graph-replayed refill rounds equal the eager ones, and inside the ban
    window no refill row takes the pad id."""
    c = MINIMIND_0P1B.with_layers(3)
    w = init_weights(c, 8, "cpu")
    rt = CandidateGroupRuntime(c, weights_to(w, "cuda"), "cuda", num_pages=1024)
    eager = CandidateGroupEngine(rt, use_graphs=False)
    graphed = CandidateGroupEngine(rt, use_graphs=True)
    prefix = _prefix(2, 32, c.vocab_size)
    base = CandidateGroupConfig(num_candidates=8, max_new_tokens=8, min_new_tokens=2,
                                sampling=SamplingParams(temperature=0.35, top_k=1, top_p=1.0),
                                max_candidates=16)
    probe = graphed.complete(prefix, base)
    graphed.reset_prefix_cache()
    # the pad id: a token the unpadded refill round takes inside the window
    window = [t for x in probe.raw_candidates[8:] for t in x.token_ids[2:]]
    assert window
    pad = max(set(window), key=window.count)
    cfg = replace(base, pad_token_id=pad)
    e = eager.complete(prefix, cfg)
    eager.reset_prefix_cache()
    g = graphed.complete(prefix, cfg)
    graphed.reset_prefix_cache()
    assert g.refill_rounds == e.refill_rounds >= 1
    assert [x.token_ids for x in g.raw_candidates] == [x.token_ids for x in e.raw_candidates]
    greedy_len = len(g.raw_candidates[0].token_ids)
    for x in g.raw_candidates[8:]:
        assert pad not in x.token_ids[2:greedy_len]
    assert rt.cache_manager.available_size == rt.num_pages


def test_graph_cache_is_bounded():
    """Captured decode graphs are kept in a least-recently-used cache of
    MAX_GRAPHS entries: many group shapes do not grow device memory without
    bound, and a re-used shape keeps its graph."""
    c = MINIMIND_0P1B.with_layers(2)
    eng, _ = _engine(c, 4, num_pages=2048, use_graphs=True)
    prefix = _prefix(4, 24, c.vocab_size)
    cap = eng.MAX_GRAPHS
    mem = []
    for t in range(2, cap + 8):
        eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=t))
        assert len(eng._graphs) <= cap
        torch.cuda.synchronize()
        mem.append(torch.cuda.memory_allocated())
    assert len(eng._graphs) == cap
    # after the cache is full, further shapes evict: memory stays at the
    # level of a full cache (plus one larger graph at most)
    per_graph = (mem[cap - 1] - mem[0]) / (cap - 1)
    assert mem[-1] <= mem[cap - 1] + 2 * max(per_graph, 1 << 20)
    # an older shape still in the cache is reused (and becomes the newest)
    key = next(k for k in eng._graphs if k[1] == cap + 3)
    g = eng._graphs[key]
    eng.complete(prefix, CandidateGroupConfig(num_candidates=8, max_new_tokens=cap + 3))
    assert next(reversed(eng._graphs)) == key and eng._graphs[key] is g
    assert len(eng._graphs) == cap
    eng.reset_prefix_cache()
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages


class _CancelAfter(CancellationToken):
    """Reads as cancelled from the n-th look on (a cancel that arrives while
    the group runs, without timing)."""

    def __init__(self, n):
        super().__init__(0)
        self.n = n
        self.looks = 0

    @property
    def cancelled(self):
        self.looks += 1
        return self.looks >= self.n


@pytest.mark.parametrize("use_graphs", [False, True])
def test_cancel_mid_group_stops_decoding(use_graphs):
    """Latest-wins cancellation is observed between decode steps
    (ime.py:971-973) in eager and graph-replayed groups: the result is
    marked cancelled, the candidates stop early, pages are all returned."""
    c = MINIMIND_0P1B.with_layers(2)
    eng, _ = _engine(c, 6, use_graphs=use_graphs)
    prefix = _prefix(6, 20, c.vocab_size)
    t = 16
    cfg = CandidateGroupConfig(num_candidates=8, max_new_tokens=t)
    full = eng.complete(prefix, cfg)
    assert not full.cancelled
    assert all(len(x.token_ids) == t for x in full.raw_candidates)
    res = eng.complete(prefix, cfg, cancellation=_CancelAfter(6))
    assert res.cancelled
    assert all(x.stop_reason == "cancelled" for x in res.raw_candidates)
    assert all(1 <= len(x.token_ids) < t // 2 for x in res.raw_candidates)
    # what was produced before the cancel is the uncancelled group's start
    for a, b in zip(res.raw_candidates, full.raw_candidates):
        assert a.token_ids == b.token_ids[: len(a.token_ids)]
    eng.reset_prefix_cache()
    assert eng.rt.cache_manager.available_size == eng.rt.num_pages
