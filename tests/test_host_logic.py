"""Host-side logic that needs no GPU: page allocator, LCP helper, candidate
selection and the engine's argument checks (CPU only)."""
from __future__ import annotations

import pytest
import torch

from aios_amd.core import Req, SamplingParams
from aios_amd.ime import (Candidate, CandidateGroupConfig, adaptive_refill_attempts,
                           candidate_valid, select_top, token_longest_common_prefix)
from aios_amd.scheduler import CacheManager
from oracle import prefix as oprefix


def test_cache_manager_order_is_deterministic():
    """python/aios/scheduler/cache.py:9-51: first-free allocation, frees appended."""
    cm = CacheManager(torch.device("cpu"), 10)
    a = cm.allocate(3)
    assert a.tolist() == [0, 1, 2] and cm.available_size == 7
    b = cm.allocate(2)
    assert b.tolist() == [3, 4]
    cm._free(a[1:])
    assert cm.available_size == 7
    assert cm.allocate(6).tolist() == [5, 6, 7, 8, 9, 1]
    assert cm.allocate(1).tolist() == [2]
    with pytest.raises(NotImplementedError):
        cm.allocate(1)


def test_cache_manager_allocate_paged():
    cm = CacheManager(torch.device("cpu"), 16)
    table = torch.full((3, 8), -1, dtype=torch.int32)
    reqs = [Req(input_ids=torch.zeros(5), cached_len=2, output_len=1, uid=0,
                sampling_params=SamplingParams(), table_idx=2),
            Req(input_ids=torch.zeros(3), cached_len=3, output_len=1, uid=1,
                sampling_params=SamplingParams(), table_idx=0)]
    cm.allocate_paged(reqs, table)
    assert table[2].tolist() == [-1, -1, 0, 1, 2, -1, -1, -1]
    assert table[0].tolist() == [-1] * 8  # extend_len 0: nothing allocated


@pytest.mark.parametrize("old,new", [([1, 2, 3], [1, 2, 3]), ([1, 2], [1, 2, 3, 4]),
                                     ([1, 2, 3, 4], [1, 2, 8]), ([5], [6]), ([], [1])])
def test_lcp_matches_oracle(old, new):
    assert token_longest_common_prefix(old, new) == oprefix.token_lcp(old, new)


def test_select_top_distinct_by_average():
    cands = [Candidate((1,), -1.0, "max_new_tokens"), Candidate((2,), -0.5, "max_new_tokens"),
             Candidate((1,), -0.1, "max_new_tokens"), Candidate((3,), -2.0, "eos"),
             Candidate((), float("-inf"), "eos")]
    top = select_top(cands, 3)
    assert [c.token_ids for c in top] == [(1,), (2,), (3,)]
    assert top[0].average_logprob == -0.1


def test_group_config_validation():
    with pytest.raises(ValueError):
        CandidateGroupConfig(num_candidates=2, display_candidates=3).validate()
    with pytest.raises(ValueError):
        CandidateGroupConfig(max_new_tokens=0).validate()
    CandidateGroupConfig().validate()


def test_req_lengths_follow_reference():
    """core.py:27-59: extend_len = device_len - cached_len; complete_one advances."""
    r = Req(input_ids=torch.zeros(7), cached_len=4, output_len=2, uid=0,
            sampling_params=SamplingParams())
    assert (r.device_len, r.extend_len, r.remain_len) == (7, 3, 2)
    r.complete_one()
    assert (r.cached_len, r.device_len, r.extend_len, r.remain_len) == (7, 8, 1, 1)


def _cands(seqs):
    return [Candidate(tuple(s), -1.0, "max_new_tokens") for s in seqs]


@pytest.mark.parametrize("seqs,used,want", [
    # 8 branches, 1 distinct: deficit 2, yield floor 1/8 -> ceil(2/0.125)=16, cap 8
    ([[1, 2, 3]] * 8, 8, 8),
    # 8 branches, 2 distinct: deficit 1, yield 1/4 -> 4 = max(2, 2, 4)
    ([[1, 2, 3]] * 7 + [[4, 5, 6]], 8, 4),
    # 2 of 2 distinct: deficit 1, yield 1 -> max(min batch 2, 2*1, 1) = 2
    ([[1, 2, 3], [4, 5, 6]], 8, 2),
    # filled: no refill
    ([[1, 1], [2, 2], [3, 3]], 8, 0),
    # budget: 22 of 24 used -> at most 2
    ([[1, 2, 3]] * 8, 22, 2),
    ([[1, 2, 3]] * 8, 24, 0),
    # empty candidates are invalid (min_new_tokens 2: one-token rows too)
    ([[], [7], [1, 2]], 8, 6),  # 1 valid of 3: ceil(2 / (1/3)) = 6
])
def test_adaptive_refill_attempts(seqs, used, want):
    """ime.py:333-370 worked by hand for display 3, budget 24, round cap 8."""
    cfg = CandidateGroupConfig(num_candidates=8, max_candidates=24, min_new_tokens=2)
    assert adaptive_refill_attempts(_cands(seqs), cfg, used) == want


def test_candidate_validity():
    cfg = CandidateGroupConfig(min_new_tokens=2)
    assert candidate_valid(Candidate((1, 2), -1.0, "eos"), cfg)
    assert not candidate_valid(Candidate((1,), -1.0, "eos"), cfg)
    assert not candidate_valid(Candidate((1, 2), -1.0, "cancelled"), cfg)
    assert not candidate_valid(Candidate((), -1.0, "eos"), CandidateGroupConfig())


@pytest.mark.parametrize("kw,msg", [
    (dict(max_candidates=4), "must cover the initial attempts"),
    (dict(max_candidates=24, refill_batch_size=0), "refill_batch_size must be positive"),
    (dict(max_candidates=24, min_refill_batch_size=9), "min_refill_batch_size"),
    (dict(max_candidates=24, refill_top_p=0.0), "refill_top_p"),
    (dict(max_candidates=24, refill_temperature=0.0), "temperatures must be positive"),
    (dict(max_candidates=24, max_refill_temperature=0.5), "max_refill_temperature"),
    (dict(max_candidates=24, refill_top_k=0), "top_k values must be positive"),
    (dict(max_candidates=24, max_refill_top_k=64), "max_refill_top_k"),
    (dict(max_candidates=24, refill_deadline_ms=-1.0), "refill_deadline_ms"),
    (dict(max_candidates=24, refill_ban_min_prefix_tokens=0), "refill_ban_min_prefix_tokens"),
    (dict(min_new_tokens=20), "min_new_tokens must be within max_new_tokens"),
])
def test_refill_config_validation(kw, msg):
    with pytest.raises(ValueError, match=msg):
        CandidateGroupConfig(num_candidates=8, **kw).validate()


def test_decode_preconditions_checker():
    """check_decode_preconditions accepts a CandidateGroup-shaped batch and
    rejects a wrong out_loc or rows that do not share the claimed prefix."""
    from aios_amd.attention import check_decode_preconditions

    prefix = [9, 4, 7]
    rows = [prefix + [20, 21], prefix + [30], prefix + [40, 41, 42]]
    indices = torch.tensor(sum(rows, []), dtype=torch.int32)
    cu_k = torch.tensor([0, 5, 9, 15], dtype=torch.int32)
    out_loc = torch.tensor([21, 30, 42], dtype=torch.int32)
    check_decode_preconditions(indices, cu_k, out_loc, 3)
    check_decode_preconditions(indices, cu_k, None, 3)
    check_decode_preconditions(indices, cu_k, out_loc, 0)
    with pytest.raises(ValueError, match="last page"):
        check_decode_preconditions(indices, cu_k, torch.tensor([21, 31, 42], dtype=torch.int32), 3)
    with pytest.raises(ValueError, match="share"):
        check_decode_preconditions(indices, cu_k, out_loc, 4)  # row 0 has 20, row 1 has 30
    bad = indices.clone()
    bad[6] = 5  # row 1's second prefix page
    with pytest.raises(ValueError, match="share"):
        check_decode_preconditions(bad, cu_k, None, 3)
    with pytest.raises(ValueError, match="exceeds"):
        check_decode_preconditions(indices, cu_k, None, 5)


def test_banned_next_ids_hand_case():
    """ime.py:977-996 worked by hand: at step 2, row 0 has produced [5, 6]
    (ban 0 = [5, 6, 7] matches -> 7), row 1 [5, 9] (no ban matches); ban 1 =
    [5, 6] is not longer than the step, so it never applies; the other
    slots hold the fill (the pad id, or -1 for none)."""
    from aios_amd.ime import banned_next_ids

    out = torch.tensor([[5, 6, -1], [5, 9, -1]])
    bans = torch.tensor([[5, 6, 7], [5, 6, -1]])
    lens = torch.tensor([3, 2])
    assert banned_next_ids(out, 2, bans, lens, 0).tolist() == [[7, 0], [0, 0]]
    assert banned_next_ids(out, 2, bans, lens, -1).tolist() == [[7, -1], [-1, -1]]
    # step 1: both rows match ban 0's first token and ban 1's
    assert banned_next_ids(out, 1, bans, lens, 3).tolist() == [[6, 6], [6, 6]]


def test_refill_ban_fill_defaults_to_the_model_pad_id():
    """The refill ban table's fill (ime.py:990-996: the tokenizer's pad id)
    comes from the group config, else from the model config's pad_token_id
    (read from and written to config.json), else none (-1)."""
    from dataclasses import replace
    from types import SimpleNamespace

    from aios_amd.config import MINIMIND_0P1B
    from aios_amd.ime import CandidateGroupConfig, CandidateGroupEngine
    from aios_amd.weights import config_from_hf, config_to_hf

    fill = CandidateGroupEngine._ban_fill
    no_pad = SimpleNamespace(rt=SimpleNamespace(config=MINIMIND_0P1B))
    with_pad = SimpleNamespace(rt=SimpleNamespace(config=replace(MINIMIND_0P1B, pad_token_id=3)))
    assert fill(no_pad, CandidateGroupConfig()) == -1
    assert fill(with_pad, CandidateGroupConfig()) == 3
    assert fill(with_pad, CandidateGroupConfig(pad_token_id=0)) == 0
    assert fill(no_pad, CandidateGroupConfig(pad_token_id=5)) == 5
    c = replace(MINIMIND_0P1B, pad_token_id=7)
    assert config_from_hf(config_to_hf(c)).pad_token_id == 7
    assert "pad_token_id" not in config_to_hf(MINIMIND_0P1B)
    assert config_from_hf(config_to_hf(MINIMIND_0P1B)).pad_token_id is None
