"""Continuous-batching scheduler with scripted models (CPU only).

The scheduler decides what every step's ragged batch looks like — which
requests, in what order, how many prompt tokens each — and that is what the
varlen/decode kernels receive.  These tests restate the reference's
scheduler tests (``tests/test_paged_greedy_generation.py``) with models
that script their next tokens and do the cache bookkeeping a real model
does (``ensure_capacity`` + ``advance``), so no kernel runs.  The known
answers are the reference's: chunk offsets 2, 4, 5; budget offsets
(2, 1, 0), (3, 1, 2), (3, 3, 3); one ragged forward over
('request-b', 'request-a') with query_start_loc (0, 2, 3).
"""

from __future__ import annotations

import pytest
import torch

from nano_infer_engine.generation import (
    ContinuousBatchingScheduler,
    GenerationConfig,
    PagedRequest,
    RequestStatus,
    TokenEvent,
    paged_greedy_generate,
    paged_prefill_chunks,
)
from nano_infer_engine.paged_cache import PagedKVCache


def _cache(num_blocks, block_size=1):
    return PagedKVCache(num_blocks, block_size, 1, 1, 1, torch.float32, "cpu")


class ScriptedModel:
    """Emits scripted next tokens; appends to the cache like a real model."""

    vocab = 16

    def __init__(self, schedules: dict[str, tuple[int, ...]], fail_decode: tuple[str, ...] = (),
                 fail_prefill: tuple[str, ...] = ()):
        self.schedules = schedules
        self.cursor = {s: 0 for s in schedules}
        self.fail_decode = fail_decode
        self.fail_prefill = fail_prefill
        self.prefill_ids: list[str] = []
        self.prefill_batches: list[int] = []
        self.decode_ids: list[tuple[str, ...]] = []
        self.ragged_calls: list[tuple[tuple[str, ...], tuple[int, ...]]] = []

    def _next(self, sid):
        # a schedule's last token repeats (chunk calls before the prompt's end
        # produce logits the scheduler never samples)
        schedule = self.schedules[sid]
        token = schedule[min(self.cursor[sid], len(schedule) - 1)]
        self.cursor[sid] += 1
        return token

    def _append(self, cache, sid, n):
        have = cache.get_sequence_length(sid)
        cache.ensure_capacity(sid, have + n)
        cache.advance(sid, n)

    def __call__(self, input_ids, *, kv_cache, sequence_id="default", sequence_ids=None):
        ids = (sequence_id,) if sequence_ids is None else tuple(sequence_ids)
        prefill = all(kv_cache.get_sequence_length(s) == 0 for s in ids)
        if prefill:
            if any(s in self.fail_prefill for s in ids):
                for s in ids:
                    if s in self.fail_prefill:
                        self._append(kv_cache, s, input_ids.shape[1])
                raise RuntimeError("prefill failed")
            self.prefill_ids.extend(ids)
            self.prefill_batches.append(len(ids))
        else:
            self.decode_ids.append(ids)
        logits = torch.zeros(len(ids), input_ids.shape[1], self.vocab)
        for row, sid in enumerate(ids):
            self._append(kv_cache, sid, input_ids.shape[1] if prefill else 1)
            logits[row, -1, self._next(sid)] = 1.0
        if not prefill and ids == self.fail_decode:
            raise RuntimeError("decode failed")
        return logits

    def forward_ragged(self, input_ids, *, kv_cache, sequence_ids, query_start_loc):
        starts = query_start_loc.tolist()
        self.ragged_calls.append((tuple(sequence_ids), tuple(starts)))
        logits = torch.zeros(input_ids.shape[0], self.vocab)
        for r, sid in enumerate(sequence_ids):
            n = starts[r + 1] - starts[r]
            self._append(kv_cache, sid, n)
            logits[starts[r + 1] - 1, self._next(sid)] = 1.0
        return logits


def _tokens(*ids):
    return torch.tensor([list(ids)])


def test_request_initial_state():
    prompt = _tokens(1, 4)
    r = PagedRequest(sequence_id="request-a", prompt=prompt)
    assert r.sequence is prompt and r.generated_tokens == 0 and not r.finished
    assert r.status is RequestStatus.PENDING and r.error is None


def test_generation_config_validation():
    with pytest.raises(ValueError, match="max_new_tokens must be positive"):
        GenerationConfig(max_new_tokens=0)
    with pytest.raises(ValueError, match="prefill_chunk_size must be positive"):
        GenerationConfig(prefill_chunk_size=0)
    with pytest.raises(TypeError, match="prefill_chunk_size must be an integer or None"):
        GenerationConfig(prefill_chunk_size=True)
    with pytest.raises(ValueError, match="requires prefill_chunk_size"):
        GenerationConfig(max_prefill_tokens_per_step=4)


def test_greedy_retires_eos_and_releases_blocks():
    model = ScriptedModel({"request-a": (2,), "request-b": (3, 4, 2), "request-c": (5, 2)})
    cache = _cache(12)
    out = paged_greedy_generate(model, (_tokens(6), _tokens(6), _tokens(6)),
                                GenerationConfig(max_new_tokens=4, eos_token_id=2), cache,
                                ("request-a", "request-b", "request-c"))
    assert tuple(s.shape[1] for s in out.sequences) == (2, 4, 3)
    assert out.generated_tokens.tolist() == [1, 3, 2]
    assert out.stopped_by_eos.all()
    assert [len(ids) for ids in model.decode_ids] == [2, 1]
    assert cache.allocator.allocated_block_count == 0


def test_greedy_admits_pending_after_eos_and_after_token_limit():
    model = ScriptedModel({"request-a": (2,), "request-b": (3, 4, 2), "request-c": (5, 2)})
    cache = _cache(8)
    out = paged_greedy_generate(model, (_tokens(6),) * 3, GenerationConfig(max_new_tokens=4, eos_token_id=2),
                                cache, ("request-a", "request-b", "request-c"), max_batch_size=2)
    assert model.prefill_ids == ["request-a", "request-b", "request-c"]
    assert model.prefill_batches == [2, 1]
    assert model.decode_ids == [("request-b",), ("request-b", "request-c")]
    assert out.generated_tokens.tolist() == [1, 3, 2]
    model = ScriptedModel({"request-a": (3, 4), "request-b": (5, 6)})
    cache = _cache(2)
    out = paged_greedy_generate(model, (_tokens(1), _tokens(1)), GenerationConfig(max_new_tokens=2), cache,
                                ("request-a", "request-b"), max_batch_size=1)
    assert model.decode_ids == [("request-a",), ("request-b",)]
    assert out.generated_tokens.tolist() == [2, 2] and not out.stopped_by_eos.any()
    assert cache.allocator.allocated_block_count == 0


def test_greedy_checks_capacity_before_prefill():
    cache = _cache(2, block_size=2)
    with pytest.raises(ValueError, match="not enough free blocks for paged generation"):
        paged_greedy_generate(ScriptedModel({}), (_tokens(1, 2), _tokens(3, 4)), GenerationConfig(max_new_tokens=2),
                              cache, ("request-a", "request-b"))
    assert cache.allocator.allocated_block_count == 0


def test_scheduler_accepts_requests_between_steps_and_emits_tokens_once():
    model = ScriptedModel({"request-a": (2,), "request-b": (3, 2), "request-c": (4, 2)})
    cache = _cache(6)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=3, eos_token_id=2), cache, max_batch_size=2)
    s.add_request("request-a", _tokens(6))
    s.add_request("request-b", _tokens(6))
    assert (s.pending_count, s.active_count) == (2, 0)
    out = s.step()
    assert out.token_events == (TokenEvent("request-a", 2), TokenEvent("request-b", 3))
    assert tuple(r.sequence_id for r in out.terminal_requests) == ("request-a",)
    s.add_request("request-c", _tokens(6))
    assert (s.pending_count, s.active_count) == (1, 1)
    assert tuple(r.sequence_id for r in s.step().terminal_requests) == ("request-b",)
    assert tuple(r.sequence_id for r in s.step().terminal_requests) == ("request-c",)
    assert not s.has_work and cache.allocator.allocated_block_count == 0

    model = ScriptedModel({"request-a": (3, 4, 2)})
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=3, eos_token_id=2), _cache(3), 1)
    request = s.add_request("request-a", _tokens(1))
    events = []
    while s.has_work:
        events.extend(s.step().token_events)
    assert events == [TokenEvent("request-a", 3), TokenEvent("request-a", 4), TokenEvent("request-a", 2)]
    assert request.sequence.tolist() == [[1, 3, 4, 2]]


def test_scheduler_isolates_prefill_and_decode_failures():
    model = ScriptedModel({"request-failed": (3,), "request-ok": (2,)}, fail_prefill=("request-failed",))
    cache = _cache(4)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=2, eos_token_id=2), cache, 2)
    bad = s.add_request("request-failed", _tokens(1))
    ok = s.add_request("request-ok", _tokens(1))
    out = s.step()
    assert out.token_events == (TokenEvent("request-ok", 2),)
    assert out.terminal_requests == (bad, ok)
    assert bad.status is RequestStatus.FAILED and isinstance(bad.error, RuntimeError)
    assert ok.status is RequestStatus.COMPLETED
    assert not s.has_work and cache.allocator.allocated_block_count == 0

    model = ScriptedModel({"request-a": (3, 4), "request-b": (5, 6), "request-c": (2,)},
                          fail_decode=("request-a", "request-b"))
    cache = _cache(6)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=3, eos_token_id=2), cache, 2)
    a, b, c = (s.add_request(x, _tokens(1)) for x in ("request-a", "request-b", "request-c"))
    out = s.step()
    assert out.token_events == (TokenEvent("request-a", 3), TokenEvent("request-b", 5))
    assert out.terminal_requests == (a, b)
    assert all(r.status is RequestStatus.FAILED for r in (a, b))
    assert s.active_count == 1 and s.reserved_blocks == c.required_blocks
    out = s.step()
    assert out.token_events == (TokenEvent("request-c", 2),) and out.terminal_requests == (c,)
    assert s.reserved_blocks == 0 and cache.allocator.allocated_block_count == 0


def test_scheduler_cancel_and_close():
    model = ScriptedModel({"request-active": (3, 4, 5), "request-pending": (6,)})
    cache = _cache(3)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=3), cache, 1)
    active = s.add_request("request-active", _tokens(1))
    pending = s.add_request("request-pending", _tokens(1))
    s.step()
    assert s.close() == (pending, active)
    assert active.status is RequestStatus.CANCELLED and pending.status is RequestStatus.CANCELLED
    assert s.is_closed and not s.has_work and s.reserved_blocks == 0
    assert cache.allocator.allocated_block_count == 0 and s.close() == ()
    with pytest.raises(RuntimeError, match="scheduler is closed"):
        s.step()
    with pytest.raises(RuntimeError, match="scheduler is closed"):
        s.add_request("request-new", _tokens(1))

    model = ScriptedModel({"request-active": (3, 4, 5), "request-pending": (6,)})
    cache = _cache(3)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=3), cache, 1)
    active = s.add_request("request-active", _tokens(1))
    pending = s.add_request("request-pending", _tokens(1))
    s.step()
    assert s.cancel_request("request-pending") and s.cancel_request("request-active")
    assert not s.cancel_request("request-active")
    assert not s.has_work and s.reserved_blocks == 0 and cache.allocator.allocated_block_count == 0

    model = ScriptedModel({"request-a": (3,)})
    cache = _cache(1)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=1), cache, 1, release_on_token_limit=False)
    request = s.add_request("request-a", _tokens(1))
    assert s.step().terminal_requests == (request,)
    assert cache.allocator.allocated_block_count == 1
    assert s.close() == () and request.status is RequestStatus.COMPLETED
    assert cache.allocator.allocated_block_count == 0


# ---------------------------------------------------------------------------
# chunked prefill: the ragged batch composition the varlen kernel receives
# ---------------------------------------------------------------------------
def test_chunked_prefill_advances_once_per_step():
    model = ScriptedModel({"request-a": (7,), "request-b": (8,)})
    cache = _cache(8)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=1, prefill_chunk_size=2), cache, 1)
    a = s.add_request("request-a", _tokens(1, 2, 3, 4, 5))
    b = s.add_request("request-b", _tokens(6))
    for offset in (2, 4):
        assert s.step().token_events == ()
        assert a.status is RequestStatus.PREFILLING and a.prefill_offset == offset
        assert cache.get_sequence_length("request-a") == offset
    out = s.step()
    assert out.token_events == () and out.terminal_requests == ()
    assert a.status is RequestStatus.ACTIVE and a.prefill_offset == 5
    out = s.step()
    assert len(out.token_events) == 1 and out.terminal_requests == (a,)
    assert b.status is RequestStatus.PENDING and s.pending_count == 1
    assert s.step().token_events == () and b.status is RequestStatus.ACTIVE
    assert s.step().terminal_requests == (b,) and not s.has_work


def test_chunked_prefill_global_budget_is_fair():
    model = ScriptedModel({f"request-{i}": (1,) for i in range(3)})
    cache = _cache(24)
    s = ContinuousBatchingScheduler(
        model, GenerationConfig(max_new_tokens=1, prefill_chunk_size=2, max_prefill_tokens_per_step=3), cache, 3
    )
    reqs = [s.add_request(f"request-{i}", _tokens(1, 2, 3, 4, 5, 6)) for i in range(3)]
    for offsets, total in (((2, 1, 0), 3), ((3, 1, 2), 6), ((3, 3, 3), 9)):
        s.step()
        assert tuple(r.prefill_offset for r in reqs) == offsets
        assert sum(cache.get_sequence_length(r.sequence_id) for r in reqs) == total


def test_prefill_chunks_then_decode_in_one_ragged_forward():
    model = ScriptedModel({"request-a": (9, 10), "request-b": (11, 12)})
    cache = _cache(12)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=2, prefill_chunk_size=2), cache, 2)
    a = s.add_request("request-a", _tokens(1))
    b = s.add_request("request-b", _tokens(2, 3, 4, 5))
    s.step()
    assert a.status is RequestStatus.ACTIVE and b.status is RequestStatus.PREFILLING
    model.ragged_calls.clear()
    out = s.step()
    assert model.ragged_calls == [(("request-b", "request-a"), (0, 2, 3))]
    assert out.token_events[0].sequence_id == "request-a"
    assert b.status is RequestStatus.ACTIVE
    # the step's plan, as the scheduler exposes it: prompt piece first, then
    # the decode row with the token just sampled
    plan = s.last_plan
    assert plan.sequence_ids == ("request-b", "request-a") and plan.query_lens == (2, 1)
    assert plan.input_ids().tolist() == [4, 5, 9]


def test_paged_prefill_chunks_returns_last_token_rows():
    model = ScriptedModel({"x": (3,), "y": (5,)})
    cache = _cache(8)
    logits = paged_prefill_chunks(model, (_tokens(1, 2, 3), _tokens(4)), cache, ("x", "y"))
    assert logits.shape == (2, ScriptedModel.vocab)
    assert logits.argmax(-1).tolist() == [3, 5]
    assert model.ragged_calls == [(("x", "y"), (0, 3, 4))]
    with pytest.raises(ValueError, match="same length"):
        paged_prefill_chunks(model, (_tokens(1),), cache, ("x", "y"))
    with pytest.raises(ValueError, match="unique"):
        paged_prefill_chunks(model, (_tokens(1), _tokens(2)), cache, ("x", "x"))
