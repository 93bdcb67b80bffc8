"""Continuous-batching scheduler over one shared paged KV cache.

Observable behaviour follows ``generation/scheduler.py:17-585`` of the
reference engine (its tests pin the token events, terminal requests, batch
order and block accounting): FIFO admission against a worst-case block
reservation of ``ceil((prompt + max_new_tokens - 1) / block_size)`` blocks;
greedy argmax of each decoding request's last logits; retirement on EOS or
on the token limit; a failed forward fails only the requests it carried;
idempotent cancel and close.

How this scheduler is organised:

* **Lanes.**  A request is in exactly one of ``pending_requests`` (FIFO),
  ``prefilling_requests`` (chunked mode: the order prompt chunks are served
  in), ``active_requests`` (decoding) or ``completed_requests``.  Terminal
  transitions all go through :meth:`_finish`, the one place that returns a
  request's block reservation and releases its cache.
* **Chunked steps** (``prefill_chunk_size`` set) are planned, run and
  committed as separate phases: :meth:`_plan_ragged_step` samples the
  decoding requests, retires the finished ones and cuts prompt pieces from
  the prefill lane under the step's token budget into a :class:`StepPlan`;
  :meth:`_run_plan` executes it as one flattened forward, prefill pieces
  first and decode rows after them (the varlen ``cu_seqlens`` layout the
  attention kernels take), or as a captured HIP-graph replay when it holds
  decode rows only (``decode_graphs=True``, a keyword this build adds);
  :meth:`_commit_plan` moves requests on.
* ``last_plan`` keeps the most recent step's plan (sequence IDs, query
  lengths and input token IDs of the forward), for tracing and for
  comparing the forward against another implementation step by step.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import torch

from nano_infer_engine.generation.config import GenerationConfig
from nano_infer_engine.generation.events import SchedulerStepOutput, TokenEvent
from nano_infer_engine.generation.paged_prefill import (
    _validate_paged_prefill_inputs,
    paged_prefill,
    paged_prefill_chunks,
)
from nano_infer_engine.generation.request import PagedRequest, RequestStatus
from nano_infer_engine.paged_cache import PagedKVCache

_LIVE = (RequestStatus.PENDING, RequestStatus.PREFILLING, RequestStatus.ACTIVE)


def reserved_block_count(prompt_length: int, max_new_tokens: int, block_size: int) -> int:
    """Blocks a request may come to occupy: its prompt plus every generated
    token but the last, which is sampled and never written to the cache."""
    return -(-(prompt_length + max_new_tokens - 1) // block_size)


@dataclass
class StepPlan:
    """One chunked step's forward: prompt pieces first, then decode rows."""

    pieces: list[tuple[PagedRequest, int, int]] = field(default_factory=list)  # (request, start, stop) of its prompt
    decode: list[PagedRequest] = field(default_factory=list)
    decode_src: torch.Tensor | None = None  # (n, 1) tokens the decode rows take their next token from
    decode_rows: list[int] = field(default_factory=list)  # the row of decode_src of each decode request
    decode_ids: list[int] = field(default_factory=list)  # the same tokens on the host

    @property
    def decode_tokens(self) -> list[torch.Tensor]:
        """The decode rows' next tokens, (1, 1) views (built when an eager
        forward needs them; a graph replay takes ``decode_ids``)."""
        return [self.decode_src[i : i + 1] for i in self.decode_rows]

    @property
    def requests(self) -> list[PagedRequest]:
        return [p[0] for p in self.pieces] + self.decode

    @property
    def sequence_ids(self) -> tuple[str, ...]:
        return tuple(r.sequence_id for r in self.requests)

    @property
    def query_lens(self) -> tuple[int, ...]:
        return tuple(stop - start for _, start, stop in self.pieces) + (1,) * len(self.decode)

    def chunks(self) -> tuple[torch.Tensor, ...]:
        """The forward's inputs, one (1, n) tensor per request, in plan order."""
        prompt_pieces = tuple(r.prompt[:, start:stop] for r, start, stop in self.pieces)
        return prompt_pieces + tuple(self.decode_tokens)

    def input_ids(self) -> torch.Tensor:
        """The forward's flattened token IDs."""
        return torch.cat([c.reshape(-1) for c in self.chunks()])


class ContinuousBatchingScheduler:
    """Schedules dynamically submitted requests over a shared paged KV cache."""

    def __init__(
        self,
        model,
        config: GenerationConfig,
        paged_cache: PagedKVCache,
        max_batch_size: int,
        *,
        release_on_token_limit: bool = True,
        decode_graphs: bool = False,
    ) -> None:
        if not config.use_cache:
            raise ValueError("continuous batching requires config.use_cache=True")
        if isinstance(max_batch_size, bool) or not isinstance(max_batch_size, int) or max_batch_size <= 0:
            raise ValueError("max_batch_size must be a positive integer")
        if not isinstance(paged_cache, PagedKVCache):
            raise TypeError("paged_cache must be a PagedKVCache")
        self.model = model
        self.config = config
        self.paged_cache = paged_cache
        self.max_batch_size = max_batch_size
        self.release_on_token_limit = release_on_token_limit
        # the cache's free blocks at construction bound every reservation
        self.block_budget = paged_cache.allocator.free_block_count
        self.reserved_blocks = 0
        self.pending_requests: deque[PagedRequest] = deque()
        self.prefilling_requests: list[PagedRequest] = []
        self.active_requests: list[PagedRequest] = []
        self.completed_requests: list[PagedRequest] = []
        self._requests: dict[str, PagedRequest] = {}
        self._closed = False
        self.last_plan: StepPlan | None = None
        self._graphs = None
        if decode_graphs:
            from nano_infer_engine.generation.decode_graph import DecodeGraphRunner

            self._graphs = DecodeGraphRunner(model, paged_cache, max_batch_size)
        # (requests of the last graph replay in order, its on-device argmax)
        self._graph_step: tuple[tuple[PagedRequest, ...], torch.Tensor] | None = None

    # ------------------------------------------------------------------ views
    @property
    def has_work(self) -> bool:
        return bool(self.pending_requests or self.prefilling_requests or self.active_requests)

    @property
    def pending_count(self) -> int:
        return len(self.pending_requests)

    @property
    def prefilling_count(self) -> int:
        return len(self.prefilling_requests)

    @property
    def active_count(self) -> int:
        return len(self.active_requests)

    @property
    def free_block_count(self) -> int:
        return self.paged_cache.allocator.free_block_count

    @property
    def is_closed(self) -> bool:
        return self._closed

    def get_request(self, sequence_id: str) -> PagedRequest:
        if sequence_id not in self._requests:
            raise KeyError(sequence_id)
        return self._requests[sequence_id]

    # -------------------------------------------------------------- lifecycle
    def _check_open(self) -> None:
        if self._closed:
            raise RuntimeError("scheduler is closed")

    def _fits(self, blocks: int) -> bool:
        return self.reserved_blocks + blocks <= self.block_budget

    def _release_cache(self, sequence_id: str) -> None:
        if self.paged_cache.has_sequence(sequence_id):
            self.paged_cache.release(sequence_id)

    def _finish(self, request: PagedRequest, status: RequestStatus, *, release: bool = True,
                error: Exception | None = None) -> None:
        """Terminal transition: return the reservation a prefilling or active
        request holds, release its cache (unless ``release`` is False) and
        record it as completed.  The caller removes it from its lane."""
        if request.status in (RequestStatus.PREFILLING, RequestStatus.ACTIVE):
            self.reserved_blocks -= request.required_blocks
        request.status = status
        if error is not None:
            request.error = error
        if release:
            self._release_cache(request.sequence_id)
        self.completed_requests.append(request)

    def _start_decoding(self, request: PagedRequest) -> None:
        """Prefill done: the request joins the decode lane (a request admitted
        without chunking takes its reservation here)."""
        if request.status is not RequestStatus.PREFILLING:
            self.reserved_blocks += request.required_blocks
        request.status = RequestStatus.ACTIVE
        self.active_requests.append(request)

    def add_request(self, sequence_id: str, prompt: torch.Tensor) -> PagedRequest:
        """Queue a request at the back of the FIFO."""
        self._check_open()
        if sequence_id in self._requests:
            raise ValueError(f"sequence ID already submitted: {sequence_id}")
        _validate_paged_prefill_inputs((prompt,), self.paged_cache, (sequence_id,))
        limit = getattr(getattr(self.model, "config", None), "max_seq_len", None)
        if limit is not None and prompt.shape[1] + self.config.max_new_tokens > limit:
            raise ValueError(f"request exceeds max model length: {sequence_id}")
        blocks = reserved_block_count(prompt.shape[1], self.config.max_new_tokens, self.paged_cache.block_size)
        if blocks > self.block_budget:
            raise ValueError(f"request cannot fit in paged cache: {sequence_id}")
        request = PagedRequest(sequence_id=sequence_id, prompt=prompt, required_blocks=blocks)
        self._requests[sequence_id] = request
        self.pending_requests.append(request)
        return request

    def add_prefilled_request(self, request: PagedRequest, last_logits: torch.Tensor) -> None:
        """Admit straight into the decode lane a request whose prompt KV is
        already in this cache (prefilled elsewhere and imported)."""
        self._check_open()
        if not isinstance(request, PagedRequest):
            raise TypeError("request must be a PagedRequest")
        if request.sequence_id in self._requests:
            raise ValueError(f"sequence ID already submitted: {request.sequence_id}")
        if request.status is not RequestStatus.PENDING:
            raise ValueError("prefilled request must have pending status")
        blocks = request.required_blocks
        if isinstance(blocks, bool) or not isinstance(blocks, int) or blocks <= 0:
            raise ValueError("prefilled request must reserve at least one block")
        if len(self.active_requests) >= self.max_batch_size:
            raise ValueError("decode batch is full")
        device = self.paged_cache.keys.device
        if request.prompt.device != device:
            raise ValueError("prefilled prompt must be on the decode cache device")
        if not isinstance(last_logits, torch.Tensor):
            raise TypeError("last_logits must be a torch.Tensor")
        if last_logits.ndim != 1:
            raise ValueError("last_logits must be a 1D tensor")
        if last_logits.device != device:
            raise ValueError("last_logits must be on the decode cache device")
        if not self._fits(blocks):
            raise ValueError("not enough reserved decode cache blocks")
        # an unknown sequence reads as length 0, which fails the length check
        if self.paged_cache.get_sequence_length(request.sequence_id) != request.prompt.shape[1]:
            raise ValueError("decode KV length must match the prompt length")
        request.last_logits = last_logits
        self._requests[request.sequence_id] = request
        self._start_decoding(request)

    def cancel_request(self, sequence_id: str) -> bool:
        """Cancel a pending, prefilling or active request (its blocks are freed).
        False if the request had already finished."""
        request = self._requests.get(sequence_id)
        if request is None:
            raise KeyError(sequence_id)
        if request.status not in _LIVE:
            return False
        lane = {
            RequestStatus.PENDING: self.pending_requests,
            RequestStatus.PREFILLING: self.prefilling_requests,
            RequestStatus.ACTIVE: self.active_requests,
        }[request.status]
        # by identity: requests are dataclasses whose == compares their tensors
        del lane[next(i for i, r in enumerate(lane) if r is request)]
        self._finish(request, RequestStatus.CANCELLED, release=request.status is not RequestStatus.PENDING)
        return True

    def close(self) -> tuple[PagedRequest, ...]:
        """Cancel every unfinished request and free every block this scheduler
        holds (also those of requests retired without a release)."""
        if self._closed:
            return ()
        self._closed = True
        unfinished = (*self.pending_requests, *self.prefilling_requests, *self.active_requests)
        for request in unfinished:
            request.status = RequestStatus.CANCELLED
        for sequence_id in self._requests:
            self._release_cache(sequence_id)
        self.pending_requests.clear()
        self.prefilling_requests.clear()
        self.active_requests.clear()
        self.reserved_blocks = 0
        self.completed_requests.extend(unfinished)
        return unfinished

    # ------------------------------------------------------------- sampling
    def _greedy_tokens(self) -> tuple[torch.Tensor, list[int], tuple[TokenEvent, ...]]:
        """Next token of every decoding request ((n, 1) device tensor, host
        list, events); one device-to-host copy for the whole lane."""
        lane = self.active_requests
        if not lane:
            empty = torch.empty((0, 1), dtype=torch.long, device=self.paged_cache.keys.device)
            return empty, [], ()
        if any(r.last_logits is None for r in lane):
            raise RuntimeError("active request is missing logits")
        tokens = self._graph_tokens()
        if tokens is None:
            tokens = torch.stack([r.last_logits for r in lane]).argmax(dim=-1, keepdim=True)
        ids = tokens.view(-1).tolist()
        for i, request in enumerate(lane):
            request.generated_tokens += 1
            request._append_row(tokens, i)
        return tokens, ids, tuple(TokenEvent(r.sequence_id, t) for r, t in zip(lane, ids))

    def _graph_tokens(self) -> torch.Tensor | None:
        """The argmax the last graph replay left on the device, when the
        decode lane is still exactly that replay's batch."""
        if self._graph_step is None:
            return None
        batch, next_ids = self._graph_step
        lane = self.active_requests
        if len(batch) != len(lane) or any(a is not b for a, b in zip(batch, lane)):
            return None
        return next_ids.clone().view(-1, 1)

    def _retire_finished(self, token_ids: list[int], terminal: list[PagedRequest]) -> list[int]:
        """Retire the decode lane's requests that sampled EOS or reached the
        token limit; returns the lane positions of the others."""
        eos = self.config.eos_token_id
        keep: list[int] = []
        for i, request in enumerate(self.active_requests):
            hit_eos = eos is not None and token_ids[i] == eos
            if not hit_eos and request.generated_tokens < self.config.max_new_tokens:
                keep.append(i)
                continue
            request.finished = hit_eos
            self._finish(request, RequestStatus.COMPLETED, release=hit_eos or self.release_on_token_limit)
            terminal.append(request)
        return keep

    def _fail(self, requests: list[PagedRequest], error: Exception, terminal: list[PagedRequest]) -> None:
        for request in requests:
            self._finish(request, RequestStatus.FAILED, error=error)
            terminal.append(request)

    # -------------------------------------------------------- chunked steps
    def _admit_to_prefill(self) -> None:
        """FIFO admission into the prefill lane while batch slots and the block
        budget allow (a request reserves its blocks when admitted)."""
        slots = self.max_batch_size - len(self.active_requests) - len(self.prefilling_requests)
        while slots > 0 and self.pending_requests and self._fits(self.pending_requests[0].required_blocks):
            request = self.pending_requests.popleft()
            request.status = RequestStatus.PREFILLING
            self.reserved_blocks += request.required_blocks
            self.prefilling_requests.append(request)
            slots -= 1

    def _cut_prompt_pieces(self) -> list[tuple[PagedRequest, int, int]]:
        """Prompt pieces of this step: requests are served from the front of
        the prefill lane, each at most ``prefill_chunk_size`` tokens, until the
        step's token budget is spent (the last piece may be shorter).  Served
        requests leave the lane; :meth:`_commit_plan` re-queues the unfinished
        ones at its back."""
        chunk = self.config.prefill_chunk_size
        budget = self.config.max_prefill_tokens_per_step
        if budget is None:  # no global budget: one chunk for every waiting request
            budget = sum(min(chunk, r.prompt.shape[1] - r.prefill_offset) for r in self.prefilling_requests)
        pieces = []
        while budget > 0 and self.prefilling_requests:
            request = self.prefilling_requests.pop(0)
            start = request.prefill_offset
            stop = start + min(chunk, request.prompt.shape[1] - start, budget)
            pieces.append((request, start, stop))
            budget -= stop - start
        return pieces

    def _plan_ragged_step(self, terminal: list[PagedRequest]) -> tuple[StepPlan, tuple[TokenEvent, ...]]:
        tokens, ids, events = self._greedy_tokens()
        keep = self._retire_finished(ids, terminal)
        plan = StepPlan(decode=[self.active_requests[i] for i in keep], decode_src=tokens, decode_rows=keep,
                        decode_ids=[ids[i] for i in keep])
        self.active_requests = list(plan.decode)
        plan.pieces = self._cut_prompt_pieces()
        return plan, events

    def _graph_eligible(self, plan: StepPlan) -> bool:
        if self._graphs is None or plan.pieces or not plan.decode:
            return False
        longest = max(self.paged_cache._lengths([r.sequence_id for r in plan.decode])) + 1
        return self._graphs.supports(len(plan.decode), longest)

    def _run_plan(self, plan: StepPlan) -> torch.Tensor:
        """The plan's forward; one logits row per planned request, in plan order."""
        self._graph_step = None
        if self._graph_eligible(plan):
            # the host IDs travel with the step's metadata copy
            logits, next_ids = self._graphs.step(None, plan.sequence_ids, host_ids=plan.decode_ids)
            self._graph_step = (tuple(plan.decode), next_ids)
            return logits
        return paged_prefill_chunks(self.model, plan.chunks(), self.paged_cache, plan.sequence_ids)

    def _commit_plan(self, plan: StepPlan, logits: torch.Tensor) -> None:
        for row, (request, _, stop) in enumerate(plan.pieces):
            request.prefill_offset = stop
            request.last_logits = logits[row]
            if stop == request.prompt.shape[1]:
                self._start_decoding(request)
            else:
                # an unfinished prompt waits behind the requests this step skipped
                self.prefilling_requests.append(request)
        for row, request in enumerate(plan.decode, start=len(plan.pieces)):
            request.last_logits = logits[row]

    def _keep_own_logits(self, plan: StepPlan) -> None:
        """A graph replay's logits rows are views of a buffer the next replay
        overwrites: requests leaving the replayed batch keep a copy."""
        if self._graph_step is None:
            return
        staying = {id(r) for r in plan.decode}
        for request in self._graph_step[0]:
            if id(request) not in staying and request.last_logits is not None:
                request.last_logits = request.last_logits.clone()

    def _step_unified_ragged(self) -> SchedulerStepOutput:
        """Prompt pieces and decode tokens in one flattened forward."""
        self._admit_to_prefill()
        if self.pending_requests and not self.active_requests and not self.prefilling_requests:
            raise RuntimeError("pending requests cannot be admitted")
        terminal: list[PagedRequest] = []
        plan, events = self._plan_ragged_step(terminal)
        self._keep_own_logits(plan)
        if plan.requests:
            self.last_plan = plan
            try:
                logits = self._run_plan(plan)
            except Exception as error:
                self._fail(plan.requests, error, terminal)
                self.active_requests = []
            else:
                self._commit_plan(plan, logits)
        return SchedulerStepOutput(events, tuple(terminal))

    # ---------------------------------------------------- unchunked steps
    def _prefill_admitted(self, terminal: list[PagedRequest]) -> None:
        """Without chunking: prefill the FIFO head requests that fit the batch
        and the block budget in one ``paged_prefill``; if that fails, prefill
        them one at a time so only a bad request fails."""
        batch: list[PagedRequest] = []
        blocks = self.reserved_blocks
        while (self.pending_requests and len(self.active_requests) + len(batch) < self.max_batch_size
               and blocks + self.pending_requests[0].required_blocks <= self.block_budget):
            batch.append(self.pending_requests.popleft())
            blocks += batch[-1].required_blocks
        if not batch:
            return
        try:
            rows = paged_prefill(self.model, tuple(r.prompt for r in batch), self.paged_cache,
                                 tuple(r.sequence_id for r in batch))
            outcomes = [(r, row, None) for r, row in zip(batch, rows)]
        except Exception:
            outcomes = []
            for request in batch:
                try:
                    row = paged_prefill(self.model, (request.prompt,), self.paged_cache, (request.sequence_id,))[0]
                    outcomes.append((request, row, None))
                except Exception as error:
                    outcomes.append((request, None, error))
        for request, row, error in outcomes:
            if error is not None:
                self._finish(request, RequestStatus.FAILED, error=error)
                terminal.append(request)
            else:
                request.last_logits = row
                self._start_decoding(request)

    def _step_unchunked(self) -> SchedulerStepOutput:
        terminal: list[PagedRequest] = []
        self._prefill_admitted(terminal)
        if not self.active_requests:
            if self.pending_requests and not self.prefilling_requests:
                raise RuntimeError("pending requests cannot be admitted")
            return SchedulerStepOutput((), tuple(terminal))
        tokens, ids, events = self._greedy_tokens()
        keep = self._retire_finished(ids, terminal)
        survivors = [self.active_requests[i] for i in keep]
        self.active_requests = survivors
        if survivors:
            try:
                logits = self.model(tokens[keep], kv_cache=self.paged_cache,
                                    sequence_ids=tuple(r.sequence_id for r in survivors))
            except Exception as error:
                self._fail(survivors, error, terminal)
                self.active_requests = []
            else:
                for row, request in enumerate(survivors):
                    request.last_logits = logits[row, -1]
        self._prefill_admitted(terminal)
        return SchedulerStepOutput(events, tuple(terminal))

    # ------------------------------------------------------------------ steps
    @torch.inference_mode()
    def step(self) -> SchedulerStepOutput:
        """One iteration: the tokens it produced and the requests it finished."""
        self._check_open()
        if self.config.prefill_chunk_size is not None:
            return self._step_unified_ragged()
        return self._step_unchunked()

    def run_until_idle(self) -> tuple[PagedRequest, ...]:
        """Step until every submitted request has finished."""
        finished: list[PagedRequest] = []
        while self.has_work:
            finished.extend(self.step().terminal_requests)
        return tuple(finished)
