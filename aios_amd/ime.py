"""CandidateGroup engine: one shared-prefix prefill, then N candidate
continuations decoded as one batch over shared prefix KV pages.

Restates the GPU control flow of ImeCompletionEngine (python/aios/ime.py):
  * token-LCP prefix reuse across keystrokes with the strict-backspace rule
    and persisted prefix pages/logits (_prepare_prefix, :1116-1168);
  * prefix prefill or LCP extension prefill (:1170-1217);
  * every candidate row of the page table starts with the same physical
    prefix pages (:1155), so the backend reads them once per kv-head
    (Batch.shared_prefix_len);
  * the branch decode loop (:891-1114) with one freshly allocated page per
    active row per step (:1219-1251), EOS compaction of active rows, and the
    suffix pages freed when the group is done (:588-592), so the pages in
    use after complete() equal the prefix length (tests/test_ime_gpu.py:36);
  * KV budget check (:467-478) and latest-wins cancellation observed once per
    decode step (:174-184, :971-973).
Candidate rule.  With ``CandidateGroupConfig.sampling`` set, the
reference's: candidate i draws every token, the first one from the prefix
logits included, with temperature / top-k / top-p from its own stateless
uniform stream keyed by (seed + i, token step), with the blocked ids
(EOS and terminal ids) forbidden before ``min_new_tokens``
(ime.py:891-1008, sample.py:12-160, on the device kernels aios_sample and
aios_stateless_uniforms).  Without it (the greedy configurations),
candidate i starts from the i-th most likely first token and then decodes
greedily (aios_greedy_select).  Either way each token's raw log-prob is
kept and candidates are ranked by average raw log-prob (the reference's
base score before text penalties, :1109-1115).  Text governance and
refill rounds are not restated (no tokenizer ships with the synthetic
models).
"""
from __future__ import annotations

import math
import threading
import time
from collections import OrderedDict
from dataclasses import dataclass, field, replace

import torch

from aios_amd import _lib
from aios_amd.config import ModelConfig
from aios_amd.core import Batch, Context, Req, SamplingParams, reset_global_ctx, set_global_ctx
from aios_amd.sample import sample_step, stateless_uniforms
from aios_amd.kvcache import MHAKVCache
from aios_amd.paged import greedy_select
from aios_amd.minimind_ime import build_causal_lm
from aios_amd.scheduler import CacheManager


def token_longest_common_prefix(left, right) -> int:
    """ime.py:165-171."""
    n = 0
    for a, b in zip(left, right):
        if a != b:
            break
        n += 1
    return n


class CancellationToken:
    """Latest-wins cancellation flag (ime.py:174-184)."""

    def __init__(self, generation_id: int) -> None:
        self.generation_id = generation_id
        self._event = threading.Event()

    def cancel(self) -> None:
        self._event.set()

    @property
    def cancelled(self) -> bool:
        return self._event.is_set()


@dataclass(frozen=True)
class CandidateGroupConfig:
    num_candidates: int = 8
    max_new_tokens: int = 16
    display_candidates: int = 3
    eos_token_id: int | None = None
    # None: greedy candidates from the top first tokens.  Otherwise the
    # reference's sampled candidates (ImeGenerationConfig defaults:
    # temperature 0.35, top_k 50, top_p 0.9, seed 20260814, ime.py:33-56).
    sampling: SamplingParams | None = None
    seed: int = 20260814
    min_new_tokens: int = 0
    blocked_token_ids: tuple[int, ...] = ()  # with EOS: forbidden before min_new_tokens
    # Adaptive refill (ime.py:333-370, 481-588): further sampled rounds while
    # fewer than display_candidates valid distinct candidates exist, up to
    # max_candidates attempts in all (0: no refill); defaults of
    # ImeGenerationConfig (ime.py:36-53).
    max_candidates: int = 0
    refill_batch_size: int = 8
    min_refill_batch_size: int = 2
    refill_temperature: float = 0.75
    refill_temperature_step: float = 0.10
    max_refill_temperature: float = 0.95
    refill_top_k: int = 96
    refill_top_k_step: int = 32
    max_refill_top_k: int = 160
    refill_top_p: float = 0.95
    refill_avoid_exact_repeats: bool = True
    refill_ban_min_prefix_tokens: int = 2
    refill_deadline_ms: float = 0.0  # no new round after this wall time (0: none)
    # Fill of the per-row banned-id table where no banned sequence matches
    # (ime.py:990-996 fills with the tokenizer's pad id, so during the ban
    # window every row is also forbidden the pad id); None: the model
    # config's pad_token_id, and no fill id if that is None too.
    pad_token_id: int | None = None

    def validate(self) -> None:
        if self.num_candidates < self.display_candidates or self.display_candidates < 1:
            raise ValueError("num_candidates must cover display_candidates")
        if self.max_new_tokens < 1:
            raise ValueError("max_new_tokens must be positive")
        if not 0 <= self.min_new_tokens <= self.max_new_tokens:
            raise ValueError("min_new_tokens must be within max_new_tokens")
        if self.max_candidates:  # refill rules (ime.py:58-96)
            if self.max_candidates < self.num_candidates:
                raise ValueError("max_sampling_attempts must cover the initial attempts")
            if self.refill_batch_size < 1:
                raise ValueError("refill_batch_size must be positive")
            if not 1 <= self.min_refill_batch_size <= self.refill_batch_size:
                raise ValueError("min_refill_batch_size must be within refill_batch_size")
            if not 0.0 < self.refill_top_p <= 1.0:
                raise ValueError("refill_top_p must be in (0, 1]")
            if self.refill_temperature <= 0.0:
                raise ValueError("IME candidate sampling temperatures must be positive")
            if self.refill_temperature_step < 0.0:
                raise ValueError("refill_temperature_step must be non-negative")
            if self.max_refill_temperature < self.refill_temperature:
                raise ValueError("max_refill_temperature must cover refill_temperature")
            if self.refill_top_k < 1:
                raise ValueError("IME candidate top_k values must be positive")
            if self.refill_top_k_step < 0:
                raise ValueError("refill_top_k_step must be non-negative")
            if self.max_refill_top_k < self.refill_top_k:
                raise ValueError("max_refill_top_k must cover refill_top_k")
            if self.refill_deadline_ms < 0.0:
                raise ValueError("refill_deadline_ms must be non-negative")
            if self.refill_ban_min_prefix_tokens < 1:
                raise ValueError("refill_ban_min_prefix_tokens must be positive")

    def blocked_ids(self) -> tuple[int, ...]:
        """ime.py:948-955: terminal ids and EOS, blocked before min_new_tokens."""
        ids = set(int(t) for t in self.blocked_token_ids)
        if self.eos_token_id is not None:
            ids.add(int(self.eos_token_id))
        return tuple(sorted(ids))


def candidate_valid(c: "Candidate", config: CandidateGroupConfig) -> bool:
    """Without a tokenizer the text filters of ime.py:187-370 reduce to: at
    least max(1, min_new_tokens) tokens and not cut off by cancellation."""
    return len(c.token_ids) >= max(1, config.min_new_tokens) and c.stop_reason != "cancelled"


def adaptive_refill_attempts(candidates, config: CandidateGroupConfig, attempts_used: int) -> int:
    """Branches for the next refill round (ime.py:333-370): enough to fill
    the Top-k deficit at the observed valid-distinct yield, at least
    min_refill_batch_size and twice the deficit, at most the round cap and
    the remaining budget."""
    remaining = config.max_candidates - attempts_used
    if remaining <= 0:
        return 0
    unique = {c.token_ids for c in candidates if candidate_valid(c, config)}
    deficit = config.display_candidates - len(unique)
    if deficit <= 0:
        return 0
    floor = 1.0 / max(1, config.refill_batch_size)
    observed = len(unique) / len(candidates) if candidates else floor
    predicted = math.ceil(deficit / max(floor, observed))
    planned = max(config.min_refill_batch_size, deficit * 2, predicted)
    return min(planned, config.refill_batch_size, remaining)


def banned_next_ids(out_ids: torch.Tensor, step: int, ban_ids: torch.Tensor,
                    ban_lens: torch.Tensor, fill: int) -> torch.Tensor:
    """Per-row forbidden ids at token index ``step`` (ime.py:977-996): for
    every banned sequence j, its token ``step`` where the row's first
    ``step`` outputs equal the sequence's and the sequence is longer than
    ``step``; ``fill`` elsewhere.  out_ids [rows, >= step], ban_ids
    [bans, >= step + 1] -> [rows, bans]."""
    match = (out_ids[:, None, :step] == ban_ids[None, :, :step]).all(-1)
    match &= ban_lens[None, :] > step
    nxt = ban_ids[None, :, step].expand(out_ids.shape[0], -1)
    return torch.where(match, nxt, torch.full_like(nxt, fill)).contiguous()


@dataclass(frozen=True)
class Candidate:
    token_ids: tuple[int, ...]
    average_logprob: float
    stop_reason: str


@dataclass
class CompletionResult:
    candidates: tuple[Candidate, ...]
    raw_candidates: tuple[Candidate, ...]
    prefix_tokens: int
    reused_prefix_tokens: int
    generated_tokens: int
    active_model_tokens: int
    latency_ms: float
    gpu_latency_ms: float
    unique_kv_pages: int
    cancelled: bool
    prefix_logits: torch.Tensor | None = field(default=None, repr=False)
    refill_rounds: int = 0
    # GPU-event time of the prefix prefill or LCP extension (0 when the
    # cached prefix logits were reused), and of the graph-replayed decode
    # steps of every round with their count (graph mode only).
    prefill_gpu_ms: float = 0.0
    replay_gpu_ms: float = 0.0
    replayed_steps: int = 0


def select_top(candidates, k: int) -> tuple[Candidate, ...]:
    """Highest average log-prob first, distinct token sequences only."""
    seen = set()
    out = []
    for c in sorted(candidates, key=lambda c: c.average_logprob, reverse=True):
        if c.token_ids in seen:
            continue
        seen.add(c.token_ids)
        out.append(c)
        if len(out) == k:
            break
    return tuple(out)


class CandidateGroupRuntime:
    """Model + paged KV pool + page allocator + global context on one GPU
    (the parts of python/aios/llm/llm.py:27-96 the IME path uses)."""

    def __init__(self, config: ModelConfig, weights: dict, device="cuda", num_pages: int = 4096,
                 max_attempts: int = 8, workspace_size: int = 8 << 20) -> None:
        from aios_amd.attention import Mi355xAttentionBackend

        self.config = config
        self.device = torch.device(device)
        self.num_pages = num_pages
        self.max_attempts = max_attempts
        backend = Mi355xAttentionBackend(config, workspace_size=workspace_size)
        self.model = build_causal_lm(config, weights, self.device, attn_backend=backend)
        self.kv_cache = MHAKVCache(config.num_kv_heads, config.num_layers, config.head_dim,
                                   num_pages, 1, torch.bfloat16, self.device)
        self.cache_manager = CacheManager(self.device, num_pages)
        reset_global_ctx()
        self.ctx = Context(page_size=1)
        self.ctx.kv_cache = self.kv_cache
        self.ctx.attn_backend = backend
        # One page-table row per candidate, as long as the rotary table; kept
        # for the runtime's life so replayed graphs see a fixed address.
        self.max_context = self.model.rotary.cos.shape[0]
        self.page_table = torch.zeros((max_attempts, self.max_context), dtype=torch.int32,
                                      device=self.device)
        self.ctx.page_table = self.page_table
        set_global_ctx(self.ctx)

    @classmethod
    def from_bundle(cls, path, device="cuda", **kw) -> "CandidateGroupRuntime":
        """A runtime over an exported weight bundle (model.safetensors +
        config.json, aios_amd.weights)."""
        from aios_amd.weights import load_bundle

        config, weights = load_bundle(path, device)
        return cls(config, weights, device, **kw)


class CandidateGroupEngine:
    """``use_graphs`` (default) replays each decode step from a HIP graph
    captured once per (rows, steps, planned prefix, KV capacity); rows that
    hit EOS are then masked instead of compacted.  ``use_graphs=False`` runs
    the eager loop with the reference's row compaction."""

    # Captured decode graphs kept at once (least recently used dropped first:
    # each holds its own memory pool, and keys grow with prefix length,
    # round size and refill sampling parameters).
    MAX_GRAPHS = 12
    # Graph-replayed steps the host queues ahead of the GPU: cancellation is
    # observed before each step is queued, so a superseded keystroke stops
    # within this many steps.
    RUN_AHEAD = 3
    # Prefills and LCP extensions of at most this many new tokens are
    # graph-replayed in graph mode (IME prompts and keystroke extensions; the
    # few-row projection kernels take up to 64 rows).
    MAX_GRAPHED_PREFILL = 64

    def __init__(self, rt: CandidateGroupRuntime, use_graphs: bool = True) -> None:
        self.rt = rt
        self.use_graphs = use_graphs
        self._graphs: OrderedDict[tuple, _DecodeGraph] = OrderedDict()
        self._prefill_graphs: OrderedDict[tuple, _PrefillGraph] = OrderedDict()
        self._generation_id = 0
        self._active: CancellationToken | None = None
        self._gen_lock = threading.Lock()
        self._run_lock = threading.Lock()
        self._prefix_ids: list[int] = []
        self._prefix_pages: torch.Tensor | None = None
        self._prefix_logits: torch.Tensor | None = None
        self._replay = [0.0, 0]  # this call's replayed-step GPU ms and count

    # -- lifecycle -------------------------------------------------------------
    def new_generation(self) -> CancellationToken:
        with self._gen_lock:
            if self._active is not None:
                self._active.cancel()
            self._generation_id += 1
            self._active = CancellationToken(self._generation_id)
            return self._active

    def reset_prefix_cache(self) -> None:
        with self._run_lock:
            if self._prefix_pages is not None and len(self._prefix_pages):
                self.rt.cache_manager._free(self._prefix_pages)
            self._prefix_ids = []
            self._prefix_pages = None
            self._prefix_logits = None

    # -- one keystroke ---------------------------------------------------------
    @torch.inference_mode()
    def complete(self, token_ids, config: CandidateGroupConfig | None = None,
                 cancellation: CancellationToken | None = None) -> CompletionResult:
        cancellation = cancellation or self.new_generation()
        with self._run_lock:
            return self._complete_locked(list(token_ids), config or CandidateGroupConfig(),
                                         cancellation)

    def _complete_locked(self, token_ids, config, cancellation) -> CompletionResult:
        wall = time.perf_counter()
        config.validate()
        if not token_ids:
            raise ValueError("prefix produced no input tokens")
        n = config.num_candidates
        if n > self.rt.max_attempts:
            raise ValueError("num_candidates exceeds the page-table rows")
        if cancellation.cancelled:
            return CompletionResult((), (), len(token_ids), 0, 0, 0,
                                    (time.perf_counter() - wall) * 1e3, 0.0, 0, True)
        p = len(token_ids)
        max_total = p + config.max_new_tokens
        if max_total > min(self.rt.config.max_position_embeddings, self.rt.max_context):
            raise ValueError("prefix + output exceeds context limit")
        rows = max(n, min(config.refill_batch_size, self.rt.max_attempts)
                   if config.max_candidates > n else 0)
        required = p + rows * max(0, config.max_new_tokens - 1)
        if required > self.rt.num_pages:
            raise ValueError(
                f"CandidateGroup KV budget is too small: need up to {required} pages, "
                f"configured {self.rt.num_pages}")
        page_table = self.rt.page_table
        self.rt.ctx.page_table = page_table
        started = torch.cuda.Event(enable_timing=True)
        ended = torch.cuda.Event(enable_timing=True)
        started.record()
        prefilled = torch.cuda.Event(enable_timing=True)
        self._replay = [0.0, 0]
        allocated: list[torch.Tensor] = []
        try:
            prefix_logits, prefix_pages, reused = self._prepare_prefix(token_ids, page_table)
            prefilled.record()
            generate = self._generate_graphed if self.use_graphs else self._generate
            raw, allocated, generated, active_tokens, cancelled = generate(
                prefix_logits, page_table, p, config, cancellation)
            unique_pages = len(prefix_pages) + sum(len(a) for a in allocated)
            if allocated:
                self.rt.cache_manager._free(torch.cat(allocated))
                allocated = []
            # Adaptive refill rounds (ime.py:504-588): the round's branch KV
            # is freed before the next round is planned.
            rounds, used = 0, n
            while not cancelled and config.max_candidates > used:
                if config.refill_deadline_ms > 0.0 and \
                        (time.perf_counter() - wall) * 1e3 >= config.refill_deadline_ms:
                    break
                attempts = min(adaptive_refill_attempts(raw, config, used), self.rt.max_attempts)
                if attempts == 0:
                    break
                rounds += 1
                sp = SamplingParams(
                    temperature=min(config.max_refill_temperature, config.refill_temperature
                                    + (rounds - 1) * config.refill_temperature_step),
                    top_k=min(config.max_refill_top_k,
                              config.refill_top_k + (rounds - 1) * config.refill_top_k_step),
                    top_p=config.refill_top_p)
                banned = []
                if config.refill_avoid_exact_repeats:
                    seen = set()
                    for c in sorted(raw, key=lambda c: c.average_logprob, reverse=True):
                        if not candidate_valid(c, config) or c.token_ids in seen:
                            continue
                        if len(c.token_ids) > config.refill_ban_min_prefix_tokens:
                            banned.append(c.token_ids)
                            seen.add(c.token_ids)
                round_cfg = replace(config, num_candidates=attempts, sampling=sp,
                                    seed=config.seed + used * 100_003)
                r_raw, r_alloc, r_gen, r_act, r_cancel = generate(
                    prefix_logits, page_table, p, round_cfg, cancellation, banned=banned)
                unique_pages = max(unique_pages, len(prefix_pages) + sum(len(a) for a in r_alloc))
                if r_alloc:
                    self.rt.cache_manager._free(torch.cat(r_alloc))
                raw += r_raw
                used += attempts
                generated += r_gen
                active_tokens += r_act
                cancelled |= r_cancel
            ended.record()
            ended.synchronize()
            return CompletionResult(
                candidates=select_top([c for c in raw if candidate_valid(c, config)]
                                      if config.max_candidates else raw,
                                      config.display_candidates),
                raw_candidates=tuple(raw),
                prefix_tokens=p,
                reused_prefix_tokens=reused,
                generated_tokens=generated,
                active_model_tokens=active_tokens + (p - reused),
                latency_ms=(time.perf_counter() - wall) * 1e3,
                gpu_latency_ms=started.elapsed_time(ended),
                unique_kv_pages=unique_pages,
                cancelled=cancelled,
                prefix_logits=prefix_logits,
                refill_rounds=rounds,
                prefill_gpu_ms=started.elapsed_time(prefilled) if reused < p else 0.0,
                replay_gpu_ms=self._replay[0],
                replayed_steps=self._replay[1],
            )
        finally:
            if allocated:
                self.rt.cache_manager._free(torch.cat(allocated))

    # -- prefix ------------------------------------------------------------------
    def _prepare_prefix(self, token_ids, page_table):
        """Token-LCP reuse of the persisted prefix (ime.py:1116-1168)."""
        old_ids, old_pages = self._prefix_ids, self._prefix_pages
        reused = token_longest_common_prefix(old_ids, token_ids)
        if old_pages is not None and self._prefix_logits is not None and \
                reused == len(old_ids) == len(token_ids):
            page_table[:, : len(token_ids)] = old_pages.unsqueeze(0)
            return self._prefix_logits, old_pages, reused
        if old_ids and reused == len(token_ids) < len(old_ids):
            reused = 0  # strict backspace: re-prefill for exact final logits
        if old_pages is not None:
            kept = old_pages[:reused]
            released = old_pages[reused:]
            if len(released):
                self.rt.cache_manager._free(released)
        else:
            kept = torch.empty(0, dtype=torch.int32, device=self.rt.device)
        ext = self.rt.cache_manager.allocate(len(token_ids) - reused)
        prefix_pages = torch.cat([kept, ext])
        page_table[:, : len(token_ids)] = prefix_pages.unsqueeze(0)
        logits = self._prefill(token_ids, reused, ext)
        self._prefix_ids = list(token_ids)
        self._prefix_pages = prefix_pages
        self._prefix_logits = logits
        return logits, prefix_pages, reused

    def _ban_fill(self, config: CandidateGroupConfig) -> int:
        """The id forbidden to rows that match no ban during the ban window:
        the group config's pad id, else the model config's, else none (-1)."""
        pad = config.pad_token_id
        if pad is None:
            pad = getattr(self.rt.config, "pad_token_id", None)
        return -1 if pad is None else int(pad)

    def _prefill(self, token_ids, cached_len: int, out_pages: torch.Tensor) -> torch.Tensor:
        """Prefix prefill (cached_len 0) or LCP extension (ime.py:1170-1217).
        With graphs, prefills of up to MAX_GRAPHED_PREFILL new tokens replay a
        graph captured per (new tokens, 64-aligned KV capacity)."""
        q_len = len(token_ids) - cached_len
        if self.use_graphs and 1 <= q_len <= self.MAX_GRAPHED_PREFILL:
            kv_cap = min(-(-len(token_ids) // 64) * 64, self.rt.max_context)
            key = (q_len, kv_cap)
            g = self._prefill_graphs.get(key)
            if g is None:
                while len(self._prefill_graphs) >= self.MAX_GRAPHS:
                    self._prefill_graphs.popitem(last=False)
                g = _PrefillGraph(self, q_len, kv_cap)
                self._prefill_graphs[key] = g
            self._prefill_graphs.move_to_end(key)
            # the graph's output buffer is overwritten by its next replay
            return g.run(token_ids, cached_len, out_pages).clone()
        dev = self.rt.device
        req = Req(input_ids=torch.empty(len(token_ids), dtype=torch.long), cached_len=cached_len,
                  output_len=1, uid=0, sampling_params=SamplingParams(max_tokens=1), table_idx=0)
        batch = Batch(reqs=[req], phase="prefill")
        batch.input_ids = torch.tensor(token_ids[cached_len:], dtype=torch.long, device=dev)
        batch.positions = torch.arange(cached_len, len(token_ids), dtype=torch.int32, device=dev)
        batch.out_loc = out_pages
        self.rt.model.attn_backend.prepare_metadata(batch)
        with self.rt.ctx.forward_batch(batch):
            return self.rt.model.forward()

    # -- candidates --------------------------------------------------------------
    def _decode_step(self, tokens: torch.Tensor, page_table, cached_len: int, rows: list[int],
                     prefix_len: int):
        """One decode forward over the active rows (ime.py:1219-1251)."""
        dev = self.rt.device
        pages = self.rt.cache_manager.allocate(len(rows))
        row_t = torch.tensor(rows, dtype=torch.long, device=dev)
        page_table[row_t, cached_len] = pages
        reqs = [Req(input_ids=torch.empty(cached_len + 1, dtype=torch.long), cached_len=cached_len,
                    output_len=1, uid=r, sampling_params=SamplingParams(max_tokens=1), table_idx=r)
                for r in rows]
        batch = Batch(reqs=reqs, phase="decode")
        batch.input_ids = tokens
        batch.positions = torch.full((len(rows),), cached_len, dtype=torch.int32, device=dev)
        batch.out_loc = pages
        batch.shared_prefix_len = prefix_len
        batch.fused_append = True  # pages[i] is row i's last page (set above)
        self.rt.model.attn_backend.prepare_metadata(batch)
        with self.rt.ctx.forward_batch(batch):
            logits = self.rt.model.forward()
        return logits, pages

    def _generate(self, prefix_logits, page_table, prefix_len: int, config, cancellation,
                  banned=()):
        """One round of n candidates (ime.py:891-1054).  ``banned``: token
        sequences a row may not reproduce -- once its output so far equals a
        banned sequence's first ``step`` tokens (step >= the ban's minimum
        prefix), that sequence's next token is forbidden for it
        (ime.py:977-1004)."""
        n = config.num_candidates
        dev = self.rt.device
        t_max = config.max_new_tokens
        out_ids = torch.full((n, t_max), -1, dtype=torch.long, device=dev)
        logp_sum = torch.zeros(n, dtype=torch.float32, device=dev)
        counts = torch.zeros(n, dtype=torch.long, device=dev)
        eos_hit = torch.zeros(n, dtype=torch.bool, device=dev)
        sampled = config.sampling is not None
        if sampled:
            uni = stateless_uniforms([config.seed + i for i in range(n)], t_max, dev)
            blocked = config.blocked_ids()
            blocked_t = (torch.tensor(blocked, dtype=torch.int32, device=dev) if blocked
                         else None)

            ban_len = max((len(b) for b in banned), default=0)
            ban_ids = ban_lens = None
            if banned:
                ban_ids = torch.full((len(banned), ban_len), -1, dtype=torch.long, device=dev)
                for i, b in enumerate(banned):
                    ban_ids[i, : len(b)] = torch.tensor(b, dtype=torch.long, device=dev)
                ban_lens = torch.tensor([len(b) for b in banned], dtype=torch.long, device=dev)

            fill = self._ban_fill(config)

            def pick(logits, rows, step):
                col = torch.full((1,), step, dtype=torch.int64, device=dev)
                by_row = None
                if banned and config.refill_ban_min_prefix_tokens <= step < ban_len:
                    by_row = banned_next_ids(out_ids[rows], step, ban_ids, ban_lens, fill)
                return sample_step(logits, config.sampling, uni[rows], col, blocked_t,
                                   config.min_new_tokens, forbidden_by_row=by_row)

            # every candidate draws its first token from the prefix logits
            token, raw_lp = pick(prefix_logits[:1].expand(n, -1), torch.arange(n, device=dev), 0)
        else:
            # First token of candidate i: the i-th most likely continuation.
            lp0 = torch.log_softmax(prefix_logits[0].float(), dim=-1)
            top = torch.topk(lp0, n)
            token = top.indices
            raw_lp = top.values
        active = list(range(n))
        allocated = []
        cancelled = False
        active_tokens = 0
        for step in range(t_max):
            if cancellation.cancelled:  # observed between steps (ime.py:971-973)
                cancelled = True
                break
            act = torch.tensor(active, dtype=torch.long, device=dev)
            if step:
                token, raw_lp = pick(logits, act, step) if sampled else greedy_select(logits)
            emitted = torch.ones_like(token, dtype=torch.bool)
            if config.eos_token_id is not None:
                emitted = token.ne(config.eos_token_id)
            out_ids[act, step] = torch.where(emitted, token, torch.full_like(token, -1))
            logp_sum[act] += torch.where(emitted, raw_lp, torch.zeros_like(raw_lp))
            counts[act] += emitted.long()
            eos_hit[act] |= ~emitted
            if step + 1 == t_max:
                break
            if config.eos_token_id is not None:
                keep = emitted.cpu().tolist()  # row compaction (ime.py:1040-1046)
                active = [r for r, k in zip(active, keep) if k]
                token = token[emitted]
                if not active:
                    break
            active_tokens += len(active)
            logits, pages = self._decode_step(token, page_table, prefix_len + step, active,
                                              prefix_len)
            allocated.append(pages)
        out_cpu = out_ids.cpu()
        cnt = counts.cpu().tolist()
        sums = logp_sum.cpu().tolist()
        eos = eos_hit.cpu().tolist()
        raw = []
        for i in range(n):
            ids = tuple(int(x) for x in out_cpu[i, : cnt[i]].tolist())
            avg = sums[i] / cnt[i] if cnt[i] else float("-inf")
            stop = "eos" if eos[i] else ("cancelled" if cancelled else "max_new_tokens")
            raw.append(Candidate(ids, avg, stop))
        return raw, allocated, int(sum(cnt)), active_tokens, cancelled

    def _generate_graphed(self, prefix_logits, page_table, prefix_len: int, config, cancellation,
                          banned=()):
        """The same candidate rule as :meth:`_generate`, with every decode step
        after the first replayed from a captured graph and no host
        synchronisation until the group is done.  ``banned`` (sampled rounds
        only, at most ``_DecodeGraph.MAX_BANS``): the banned-repeat rule of
        :meth:`_generate`, evaluated on the device each step."""
        if banned and (config.sampling is None or len(banned) > _DecodeGraph.MAX_BANS):
            return self._generate(prefix_logits, page_table, prefix_len, config, cancellation,
                                  banned=banned)
        n = config.num_candidates
        t_max = config.max_new_tokens
        if cancellation.cancelled:
            return ([Candidate((), float("-inf"), "cancelled") for _ in range(n)], [], 0, 0, True)
        # Plan the prefix in multiples of 64 and the KV capacity up to the next
        # multiple of 64, so neighbouring prefix lengths share one graph.
        plan_prefix = (prefix_len // 64) * 64
        kv_cap = min(-(-(prefix_len + t_max) // 64) * 64, self.rt.max_context)
        sp = config.sampling
        key = (n, t_max, plan_prefix, kv_cap, config.eos_token_id,
               None if sp is None else (sp.temperature, sp.top_k, sp.top_p),
               config.min_new_tokens, config.blocked_ids(),
               (config.refill_ban_min_prefix_tokens, config.pad_token_id) if banned else None)
        g = self._graphs.get(key)
        if g is None:
            while len(self._graphs) >= self.MAX_GRAPHS:
                self._graphs.popitem(last=False)  # drops the graph and its pool
            g = _DecodeGraph(self, n, t_max, plan_prefix, kv_cap, config.eos_token_id, config,
                             bans=bool(banned))
            self._graphs[key] = g
        self._graphs.move_to_end(key)
        if banned:
            g.set_bans(banned)
        allocated = []
        if t_max > 1:
            pages = self.rt.cache_manager.allocate(n * (t_max - 1))
            allocated.append(pages)
            g.pages[: t_max - 1].copy_(pages.view(t_max - 1, n))
        g.start(prefix_logits, prefix_len, config.seed)
        cancelled = False
        queued: list[torch.cuda.Event] = []
        first, last = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        first.record()
        for i in range(t_max - 1):
            # Observed between steps (ime.py:971-973): the host waits until at
            # most RUN_AHEAD steps are queued, so a cancel stops the group
            # within that many steps instead of after every step was queued.
            if i >= self.RUN_AHEAD:
                queued[i - self.RUN_AHEAD].synchronize()
            if cancellation.cancelled:
                cancelled = True
                break
            g.run_step()
            ev = torch.cuda.Event()
            ev.record()
            queued.append(ev)
        last.record()
        ids = g.out_ids.cpu()
        cnt = g.counts.cpu().tolist()
        sums = g.logp_sum.cpu().tolist()
        eos = g.eos_hit.cpu().tolist()
        fed = int(g.fed.item())
        self._replay[0] += first.elapsed_time(last)
        self._replay[1] += len(queued)
        raw = []
        for i in range(n):
            row = tuple(int(x) for x in ids[i][ids[i] >= 0].tolist())
            avg = sums[i] / cnt[i] if cnt[i] else float("-inf")
            stop = "eos" if eos[i] else ("cancelled" if cancelled else "max_new_tokens")
            raw.append(Candidate(row, avg, stop))
        return raw, allocated, int(sum(cnt)), fed, cancelled


class _PrefillGraph:
    """Fixed buffers and the captured forward of one prefill shape: ``q_len``
    new tokens of page-table row 0 against at most ``kv_cap`` positions
    (cached + new).  One replay rebuilds the request's KV length and page
    indices on the device, runs the model (the new tokens' K/V written to
    their pages) and leaves the last token's logits in ``logits``."""

    def __init__(self, eng: "CandidateGroupEngine", q_len: int, kv_cap: int) -> None:
        rt = eng.rt
        dev = rt.device
        self.rt = rt
        self.q_len = q_len
        self.ids = torch.zeros(q_len, dtype=torch.long, device=dev)
        self.pos = torch.zeros(q_len, dtype=torch.int32, device=dev)
        self.ramp = torch.arange(q_len, dtype=torch.int32, device=dev)
        self.kv_len = torch.zeros(1, dtype=torch.int32, device=dev)
        self.out_loc = torch.zeros(q_len, dtype=torch.int32, device=dev)
        self.md = rt.model.attn_backend.prepare_static_prefill(q_len, kv_cap, rt.page_table, 0)
        req = Req(input_ids=torch.empty(q_len, dtype=torch.long), cached_len=0, output_len=1,
                  uid=0, sampling_params=SamplingParams(max_tokens=1), table_idx=0)
        self.batch = Batch(reqs=[req], phase="prefill")
        self.batch.input_ids = self.ids
        self.batch.positions = self.pos
        self.batch.out_loc = self.out_loc
        self.batch.attn_metadata = self.md
        self.graph: torch.cuda.CUDAGraph | None = None
        self.logits: torch.Tensor | None = None

    def _body(self) -> torch.Tensor:
        self.md.refresh(self.kv_len)
        with self.rt.ctx.forward_batch(self.batch):
            return self.rt.model.forward()

    def run(self, token_ids, cached_len: int, out_pages: torch.Tensor) -> torch.Tensor:
        if len(token_ids) - cached_len != self.q_len or out_pages.numel() != self.q_len:
            raise ValueError("prefill graph used with another number of new tokens")
        self.ids.copy_(torch.tensor(token_ids[cached_len:], dtype=torch.long))
        torch.add(self.ramp, cached_len, out=self.pos)
        self.kv_len.fill_(len(token_ids))
        self.out_loc.copy_(out_pages)
        if self.graph is not None:
            self.graph.replay()
            return self.logits
        # First use: run eagerly on the capture stream (which also warms every
        # library call there), then capture for the next ones.
        dev = self.rt.device
        cur = torch.cuda.current_stream(dev)
        stream = torch.cuda.Stream(dev)
        stream.wait_stream(cur)
        with torch.cuda.stream(stream):
            out = self._body()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self.logits = self._body()
        cur.wait_stream(stream)
        self.graph = graph
        return out


class _DecodeGraph:
    """Fixed buffers and the captured decode step of one CandidateGroup shape.

    State on the device: ``tokens`` (the token each row feeds next), ``pos``
    (its position), ``step`` (index of the fed token), the pre-allocated
    pages of every step (``pages[s]`` receives the K/V of step s, the order
    in which the reference allocates one page per row per step), outputs and
    score sums.  One replay writes the page-table column, refreshes the
    decode metadata, runs the model, takes the argmax and advances the state.
    """

    MAX_BANS = 32  # banned sequences a refill-round graph holds

    def __init__(self, eng: "CandidateGroupEngine", rows: int, steps: int, plan_prefix: int,
                 kv_cap: int, eos: int | None, config: CandidateGroupConfig,
                 bans: bool = False) -> None:
        rt = eng.rt
        dev = rt.device
        self.rt = rt
        self.rows = rows
        self.steps = steps
        self.eos = eos
        # sampled candidates: the group's uniform table (refilled per group),
        # the ids blocked before min_new_tokens
        self.sampling = config.sampling
        self.min_new = config.min_new_tokens
        blocked = config.blocked_ids()
        self.blocked = (torch.tensor(blocked, dtype=torch.int32, device=dev) if blocked
                        else None)
        self.uni = torch.zeros((rows, steps), dtype=torch.float32, device=dev)
        self.tokens = torch.zeros(rows, dtype=torch.long, device=dev)
        self.pos = torch.zeros(rows, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.long, device=dev)
        self.pages = torch.zeros((max(steps - 1, 1), rows), dtype=torch.int32, device=dev)
        self.out_ids = torch.full((rows, steps), -1, dtype=torch.long, device=dev)
        self.logp_sum = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.counts = torch.zeros(rows, dtype=torch.long, device=dev)
        self.finished = torch.zeros(rows, dtype=torch.bool, device=dev)
        self.eos_hit = torch.zeros(rows, dtype=torch.bool, device=dev)
        self.fed = torch.zeros(1, dtype=torch.long, device=dev)
        self.row_ids = torch.arange(rows, dtype=torch.long, device=dev)
        self.out_loc = torch.zeros(rows, dtype=torch.int32, device=dev)
        # Banned repeats of a refill round (ime.py:977-1004): -1-padded
        # sequences, their lengths (0: unused slot) and the minimum prefix.
        self.bans = bans
        if bans:
            self.ban_ids = torch.full((self.MAX_BANS, steps), -1, dtype=torch.long, device=dev)
            self.ban_lens = torch.zeros(self.MAX_BANS, dtype=torch.long, device=dev)
            self.ban_cols = torch.arange(steps, dtype=torch.long, device=dev)
            self.ban_min = torch.full((1,), config.refill_ban_min_prefix_tokens,
                                      dtype=torch.long, device=dev)
            self.ban_fill = eng._ban_fill(config)
            self.ban_max = torch.zeros(1, dtype=torch.long, device=dev)  # longest ban
        self.tok = torch.zeros(rows, dtype=torch.long, device=dev)
        self.raw = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.step_next = torch.zeros(1, dtype=torch.long, device=dev)  # step + 1, per replay
        self.md = rt.model.attn_backend.prepare_static_decode(self.row_ids, kv_cap, plan_prefix,
                                                              rt.page_table)
        # The step's preparation also gathers the embedding rows for a model
        # that takes them (the standard trunk; the Block-AttnRes trunk
        # gathers into its depth bank itself).
        emb = rt.model.w["embed"]
        self.h_in = (torch.empty((rows, emb.shape[1]), dtype=emb.dtype, device=dev)
                     if getattr(rt.model, "takes_input_embeds", False) else None)
        reqs = [Req(input_ids=torch.empty(1), cached_len=0, output_len=1, uid=r,
                    sampling_params=SamplingParams(max_tokens=1), table_idx=r)
                for r in range(rows)]
        self.batch = Batch(reqs=reqs, phase="decode")
        # aios_cg_step_prepare writes each row's page into both out_loc and the
        # page-table column the step attends to last
        self.batch.fused_append = True
        self.batch.input_ids = self.tokens
        self.batch.input_embeds = self.h_in
        self.batch.positions = self.pos
        self.batch.attn_metadata = self.md
        self.graph: torch.cuda.CUDAGraph | None = None

    def set_bans(self, banned) -> None:
        ids = torch.full((self.MAX_BANS, self.steps), -1, dtype=torch.long)
        lens = torch.zeros(self.MAX_BANS, dtype=torch.long)
        for i, b in enumerate(banned):
            b = b[: self.steps]
            ids[i, : len(b)] = torch.tensor(b, dtype=torch.long)
            lens[i] = len(b)
        self.ban_ids.copy_(ids)
        self.ban_lens.copy_(lens)
        self.ban_max.fill_(int(lens.max()))

    def _banned_next(self) -> torch.Tensor:
        """Per-row forbidden ids of the token being sampled (index step + 1):
        a ban's next token where the row's output so far equals the ban's
        prefix of that length, from the minimum prefix on; the pad id (or
        -1, none) elsewhere while a ban is that long (ime.py:977-996), -1
        outside that window."""
        s = self.step_next
        eq = (self.out_ids[:, None, :] == self.ban_ids[None, :, :]) | \
            (self.ban_cols >= s)[None, None, :]
        window = (s >= self.ban_min) & (s < self.ban_max)
        match = eq.all(-1) & (self.ban_lens > s)[None, :] & window[None, :]
        nxt = self.ban_ids.index_select(1, s).view(1, -1).expand(self.rows, -1)
        fill = torch.where(window, self.ban_fill, -1).view(1, 1)
        return torch.where(match, nxt, fill.expand_as(nxt)).contiguous()

    def start(self, prefix_logits: torch.Tensor, prefix_len: int, seed: int) -> None:
        """Step 0: candidate i samples the prefix logits with its own uniform
        stream (sampled candidates), or takes the i-th most likely first
        token (greedy candidates)."""
        if self.sampling is not None:
            dev = self.rt.device
            self.uni.copy_(stateless_uniforms([seed + i for i in range(self.rows)], self.steps,
                                              dev))
            col = torch.zeros(1, dtype=torch.int64, device=dev)
            tok, val = sample_step(prefix_logits[:1].expand(self.rows, -1), self.sampling,
                                   self.uni, col, self.blocked, self.min_new)
        else:
            lp0 = torch.log_softmax(prefix_logits[0].float(), dim=-1)
            top = torch.topk(lp0, self.rows)
            tok, val = top.indices, top.values
        emitted = torch.ones_like(tok, dtype=torch.bool) if self.eos is None else tok.ne(self.eos)
        self.tokens.copy_(tok)
        self.out_ids.fill_(-1)
        self.out_ids[:, 0] = torch.where(emitted, tok, torch.full_like(tok, -1))
        self.logp_sum.copy_(torch.where(emitted, val, torch.zeros_like(val)))
        self.counts.copy_(emitted.long())
        self.finished.copy_(~emitted)
        self.eos_hit.copy_(~emitted)
        self.fed.zero_()
        self.pos.fill_(prefix_len)
        self.step.zero_()

    def _body(self) -> None:
        """One step: the page-table column, decode metadata, step column and
        embedding rows (aios_cg_step_prepare), model, pick, then the state
        update (aios_cg_step_end) -- the ime.py:1010-1054 bookkeeping in two
        launches."""
        rt = self.rt
        lib = _lib.lib()
        pt = rt.page_table
        md = self.md
        stream = torch.cuda.current_stream(self.rt.device).cuda_stream
        emb = rt.model.w["embed"]
        _lib.check(lib.aios_cg_step_prepare(
            self.step.data_ptr(), self.pages.data_ptr(), self.pages.shape[0], self.rows,
            self.out_loc.data_ptr(), pt.data_ptr(), pt.stride(0), pt.shape[1],
            self.pos.data_ptr(), md.cu_seqlens_k_gpu.data_ptr(), md.indices.data_ptr(),
            md.max_kv_len, self.step_next.data_ptr(), self.tokens.data_ptr(),
            emb.data_ptr() if self.h_in is not None else None, emb.shape[0], emb.shape[1],
            self.h_in.data_ptr() if self.h_in is not None else None, stream),
            "aios_cg_step_prepare")
        self.batch.out_loc = self.out_loc
        with rt.ctx.forward_batch(self.batch):
            logits = rt.model.forward()
        if self.sampling is not None:
            tok, raw = sample_step(logits, self.sampling, self.uni, self.step_next, self.blocked,
                                   self.min_new, forbidden_by_row=(self._banned_next() if self.bans
                                                                   else None),
                                   out=(self.tok, self.raw))
        else:
            tok, raw = greedy_select(logits, out=(self.tok, self.raw))
        _lib.check(lib.aios_cg_step_end(
            self.step.data_ptr(), self.rows, tok.data_ptr(), raw.data_ptr(),
            -1 if self.eos is None else int(self.eos), self.finished.data_ptr(),
            self.eos_hit.data_ptr(), self.out_ids.data_ptr(), self.out_ids.stride(0),
            self.out_ids.shape[1], self.logp_sum.data_ptr(), self.counts.data_ptr(),
            self.tokens.data_ptr(), self.pos.data_ptr(), self.fed.data_ptr(), stream),
            "aios_cg_step_end")

    def run_step(self) -> None:
        if self.graph is not None:
            self.graph.replay()
            return
        # First use: run this step eagerly on the capture stream (which also
        # warms every library call there), then capture it for the next ones.
        dev = self.rt.device
        cur = torch.cuda.current_stream(dev)
        stream = torch.cuda.Stream(dev)
        stream.wait_stream(cur)
        with torch.cuda.stream(stream):
            self._body()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self._body()
        cur.wait_stream(stream)
        self.graph = graph
