"""Continuous-batching scheduler over one shared paged KV cache.

Behaviour of ``generation/scheduler.py:17-585`` of the reference engine:
FIFO admission with worst-case block reservation
``ceil((prompt + max_new_tokens - 1) / block_size)``; greedy argmax of each
active request's last logits; EOS / token-limit retirement; request-level
failure isolation; idempotent cancel/close.  With ``prefill_chunk_size`` set,
every step is one flattened forward over ``[prefill chunks..., decode
tokens...]`` (prefill first), chunks picked round-robin under the global
``max_prefill_tokens_per_step`` budget — this is what feeds the varlen
paged-attention path.

With ``decode_graphs=True`` (a keyword this build adds) a step that carries
only decode tokens replays a captured HIP graph of the whole model step
(:mod:`nano_infer_engine.generation.decode_graph`), which also leaves the
next greedy tokens on the device; every other step runs eagerly.
"""

from __future__ import annotations

from collections import deque

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
        self.block_budget = paged_cache.allocator.free_block_count
        self.pending_requests: deque[PagedRequest] = deque()
        self.prefilling_requests: list[PagedRequest] = []
        self.active_requests: list[PagedRequest] = []
        self.completed_requests: list[PagedRequest] = []
        self.reserved_blocks = 0
        self._requests: dict[str, PagedRequest] = {}
        self._closed = False
        self._graphs = None
        if decode_graphs:
            from nano_infer_engine.generation.decode_graph import DecodeGraphRunner

            self._graphs = DecodeGraphRunner(model, paged_cache, max_batch_size)
        # requests of the last graph step, in order, and its argmax (device)
        self._graph_step: tuple[tuple[PagedRequest, ...], torch.Tensor] | None = None

    # ------------------------------------------------------------------ state
    @property
    def has_work(self) -> bool:
        return bool(self.pending_requests or self.prefilling_requests or self.active_requests)

    @property
    def pending_count(self) -> int:
        return len(self.pending_requests)

    @property
    def active_count(self) -> int:
        return len(self.active_requests)

    @property
    def prefilling_count(self) -> int:
        return len(self.prefilling_requests)

    @property
    def free_block_count(self) -> int:
        return self.paged_cache.allocator.free_block_count

    @property
    def is_closed(self) -> bool:
        return self._closed

    def get_request(self, sequence_id: str) -> PagedRequest:
        try:
            return self._requests[sequence_id]
        except KeyError:
            raise KeyError(sequence_id) from None

    # -------------------------------------------------------------- requests
    def _blocks_reserved_for(self, prompt_len: int) -> int:
        bs = self.paged_cache.block_size
        return (prompt_len + self.config.max_new_tokens - 1 + bs - 1) // bs

    def add_request(self, sequence_id: str, prompt: torch.Tensor) -> PagedRequest:
        """Queue a request (FIFO)."""
        if self._closed:
            raise RuntimeError("scheduler is closed")
        if sequence_id in self._requests:
            raise ValueError(f"sequence ID already submitted: {sequence_id}")
        _validate_paged_prefill_inputs((prompt,), self.paged_cache, (sequence_id,))
        max_model_len = getattr(getattr(self.model, "config", None), "max_seq_len", None)
        if max_model_len is not None and prompt.shape[1] + self.config.max_new_tokens > max_model_len:
            raise ValueError(f"request exceeds max model length: {sequence_id}")
        required = self._blocks_reserved_for(prompt.shape[1])
        if required > self.block_budget:
            raise ValueError(f"request cannot fit in paged cache: {sequence_id}")
        request = PagedRequest(sequence_id=sequence_id, prompt=prompt, required_blocks=required)
        self.pending_requests.append(request)
        self._requests[sequence_id] = request
        return request

    def add_prefilled_request(self, request: PagedRequest, last_logits: torch.Tensor) -> None:
        """Admit a request whose KV is already in this cache (prefilled elsewhere)."""
        if self._closed:
            raise RuntimeError("scheduler is closed")
        if not isinstance(request, PagedRequest):
            raise TypeError("request must be a PagedRequest")
        if request.sequence_id in self._requests:
            raise ValueError(f"sequence ID already submitted: {request.sequence_id}")
        if request.status is not RequestStatus.PENDING:
            raise ValueError("prefilled request must have pending status")
        rb = request.required_blocks
        if isinstance(rb, bool) or not isinstance(rb, int) or rb <= 0:
            raise ValueError("prefilled request must reserve at least one block")
        if len(self.active_requests) >= self.max_batch_size:
            raise ValueError("decode batch is full")
        if request.prompt.device != self.paged_cache.keys.device:
            raise ValueError("prefilled prompt must be on the decode cache device")
        if not isinstance(last_logits, torch.Tensor):
            raise TypeError("last_logits must be a torch.Tensor")
        if last_logits.ndim != 1:
            raise ValueError("last_logits must be a 1D tensor")
        if last_logits.device != self.paged_cache.keys.device:
            raise ValueError("last_logits must be on the decode cache device")
        if self.reserved_blocks + rb > self.block_budget:
            raise ValueError("not enough reserved decode cache blocks")
        # an unknown sequence reads as length 0 and fails the length check
        if self.paged_cache.get_sequence_length(request.sequence_id) != request.prompt.shape[1]:
            raise ValueError("decode KV length must match the prompt length")
        request.last_logits = last_logits
        request.status = RequestStatus.ACTIVE
        self.active_requests.append(request)
        self.reserved_blocks += rb
        self._requests[request.sequence_id] = request

    def _release_request_cache(self, sequence_id: str) -> None:
        if self.paged_cache.has_sequence(sequence_id):
            self.paged_cache.release(sequence_id)

    def _activate(self, request: PagedRequest) -> None:
        request.status = RequestStatus.ACTIVE
        self.active_requests.append(request)
        self.reserved_blocks += request.required_blocks

    def _admit_pending_requests(self) -> list[PagedRequest]:
        """Non-chunked admission: prefill as many FIFO requests as fit."""
        if self.config.prefill_chunk_size is not None:
            self._admit_chunked_requests()
            return []
        admitted: list[PagedRequest] = []
        reserved = self.reserved_blocks
        while self.pending_requests and len(self.active_requests) + len(admitted) < self.max_batch_size:
            head = self.pending_requests[0]
            if reserved + head.required_blocks > self.block_budget:
                break
            admitted.append(self.pending_requests.popleft())
            reserved += head.required_blocks
        if not admitted:
            return []
        try:
            logits = paged_prefill(
                self.model,
                tuple(r.prompt for r in admitted),
                self.paged_cache,
                tuple(r.sequence_id for r in admitted),
            )
        except Exception:
            # Retry one by one so a bad prompt fails only its own request.
            failed: list[PagedRequest] = []
            for request in admitted:
                try:
                    single = paged_prefill(self.model, (request.prompt,), self.paged_cache, (request.sequence_id,))
                except Exception as error:
                    self._release_request_cache(request.sequence_id)
                    request.status = RequestStatus.FAILED
                    request.error = error
                    failed.append(request)
                    continue
                request.last_logits = single[0]
                self._activate(request)
            return failed
        for request, row in zip(admitted, logits):
            request.last_logits = row
            self._activate(request)
        return []

    def _admit_chunked_requests(self) -> None:
        occupied = len(self.active_requests) + len(self.prefilling_requests)
        while self.pending_requests and occupied < self.max_batch_size:
            head = self.pending_requests[0]
            if self.reserved_blocks + head.required_blocks > self.block_budget:
                break
            self.pending_requests.popleft()
            head.status = RequestStatus.PREFILLING
            self.prefilling_requests.append(head)
            self.reserved_blocks += head.required_blocks
            occupied += 1

    def _take_prefill_chunks(self) -> tuple[list[PagedRequest], tuple[torch.Tensor, ...]]:
        chunk_size = self.config.prefill_chunk_size
        assert chunk_size is not None
        budget = self.config.max_prefill_tokens_per_step
        if budget is None:
            budget = sum(min(chunk_size, r.prompt.shape[1] - r.prefill_offset) for r in self.prefilling_requests)
        scheduled: list[PagedRequest] = []
        chunks: list[torch.Tensor] = []
        while self.prefilling_requests and budget > 0:
            request = self.prefilling_requests.pop(0)
            start = request.prefill_offset
            take = min(chunk_size, request.prompt.shape[1] - start, budget)
            chunks.append(request.prompt[:, start : start + take])
            scheduled.append(request)
            budget -= take
        return scheduled, tuple(chunks)

    def _finish_prefill_chunks(self, scheduled, chunks, logits) -> None:
        for request, row, chunk in zip(scheduled, logits, chunks):
            request.prefill_offset += chunk.shape[1]
            request.last_logits = row
            if request.prefill_offset == request.prompt.shape[1]:
                request.status = RequestStatus.ACTIVE
                self.active_requests.append(request)
            else:
                # unfinished chunks rotate behind the requests that waited
                self.prefilling_requests.append(request)

    def cancel_request(self, sequence_id: str) -> bool:
        """Cancel a pending, prefilling or active request and free its blocks."""
        request = self._requests.get(sequence_id)
        if request is None:
            raise KeyError(sequence_id)
        status = request.status
        if status is RequestStatus.PENDING:
            self.pending_requests = deque(r for r in self.pending_requests if r is not request)
        elif status is RequestStatus.PREFILLING:
            self.prefilling_requests = [r for r in self.prefilling_requests if r is not request]
            self.reserved_blocks -= request.required_blocks
            self._release_request_cache(sequence_id)
        elif status is RequestStatus.ACTIVE:
            self.active_requests = [r for r in self.active_requests if r is not request]
            self.reserved_blocks -= request.required_blocks
            self._release_request_cache(sequence_id)
        else:
            return False
        request.status = RequestStatus.CANCELLED
        self.completed_requests.append(request)
        return True

    def close(self) -> tuple[PagedRequest, ...]:
        """Cancel all unfinished requests and free every scheduler-owned block."""
        if self._closed:
            return ()
        self._closed = True
        cancelled = [*self.pending_requests, *self.prefilling_requests, *self.active_requests]
        for request in cancelled:
            request.status = RequestStatus.CANCELLED
        for request in self._requests.values():
            self._release_request_cache(request.sequence_id)
        self.pending_requests.clear()
        self.prefilling_requests.clear()
        self.active_requests.clear()
        self.reserved_blocks = 0
        self.completed_requests.extend(cancelled)
        return tuple(cancelled)

    # ------------------------------------------------------------------ steps
    def _graph_argmax(self) -> torch.Tensor | None:
        """The last graph step's argmax, if the active requests are exactly that step's, in order."""
        if self._graph_step is None:
            return None
        requests, next_ids = self._graph_step
        active = self.active_requests
        if len(requests) != len(active) or any(a is not b for a, b in zip(requests, active)):
            return None
        return next_ids.clone().view(-1, 1)

    def _sample_active(self) -> tuple[torch.Tensor, list[int], tuple[TokenEvent, ...]]:
        """Greedy next token of every active request (one device->host sync)."""
        rows = []
        for request in self.active_requests:
            if request.last_logits is None:
                raise RuntimeError("active request is missing logits")
            rows.append(request.last_logits)
        if rows:
            next_tokens = self._graph_argmax()
            if next_tokens is None:
                next_tokens = torch.stack(rows).argmax(dim=-1, keepdim=True)
            token_ids = next_tokens.squeeze(-1).tolist()
        else:
            next_tokens = torch.empty((0, 1), dtype=torch.long, device=self.paged_cache.keys.device)
            token_ids = []
        events = tuple(TokenEvent(r.sequence_id, token_ids[i]) for i, r in enumerate(self.active_requests))
        for i, request in enumerate(self.active_requests):
            request.generated_tokens += 1
            request.append_token(next_tokens[i : i + 1])
        return next_tokens, token_ids, events

    def _retire(self, token_ids: list[int], completed: list[PagedRequest]) -> list[int]:
        """Retire finished active requests; return the indices of the survivors."""
        eos = self.config.eos_token_id
        survivors: list[int] = []
        for i, request in enumerate(self.active_requests):
            by_eos = eos is not None and token_ids[i] == eos
            if by_eos or request.generated_tokens >= self.config.max_new_tokens:
                request.finished = by_eos
                request.status = RequestStatus.COMPLETED
                self.reserved_blocks -= request.required_blocks
                if by_eos or self.release_on_token_limit:
                    self._release_request_cache(request.sequence_id)
                completed.append(request)
            else:
                survivors.append(i)
        return survivors

    def _fail_all(self, requests: list[PagedRequest], error: Exception, completed: list[PagedRequest]) -> None:
        for request in requests:
            request.status = RequestStatus.FAILED
            request.error = error
            self.reserved_blocks -= request.required_blocks
            self._release_request_cache(request.sequence_id)
            completed.append(request)
        self.active_requests = []

    def _step_unified_ragged(self) -> SchedulerStepOutput:
        """Chunked prefill and decode tokens in one flattened forward."""
        self._admit_chunked_requests()
        if not self.active_requests and not self.prefilling_requests and self.pending_requests:
            raise RuntimeError("pending requests cannot be admitted")
        completed: list[PagedRequest] = []
        next_tokens, token_ids, events = self._sample_active()
        keep = self._retire(token_ids, completed)
        survivors = [self.active_requests[i] for i in keep]
        survivor_tokens = [next_tokens[i : i + 1] for i in keep]
        self.active_requests = survivors

        prefill_requests, prefill_chunks = self._take_prefill_chunks()
        ragged_requests = [*prefill_requests, *survivors]
        self._detach_graph_logits(survivors)
        if ragged_requests:
            try:
                if self._use_graph(prefill_requests, survivors):
                    logits, next_ids = self._graphs.step(
                        torch.cat(survivor_tokens).view(-1), tuple(r.sequence_id for r in survivors)
                    )
                    self._graph_step = (tuple(survivors), next_ids)
                else:
                    logits = paged_prefill_chunks(
                        self.model,
                        (*prefill_chunks, *survivor_tokens),
                        self.paged_cache,
                        tuple(r.sequence_id for r in ragged_requests),
                    )
            except Exception as error:
                self._fail_all(ragged_requests, error, completed)
            else:
                n = len(prefill_requests)
                self._finish_prefill_chunks(prefill_requests, prefill_chunks, logits[:n])
                for request, row in zip(survivors, logits[n:]):
                    request.last_logits = row
        self.completed_requests.extend(completed)
        return SchedulerStepOutput(events, tuple(completed))

    def _use_graph(self, prefill_requests: list[PagedRequest], survivors: list[PagedRequest]) -> bool:
        self._graph_step = None
        if self._graphs is None or prefill_requests or not survivors:
            return False
        longest = max(self.paged_cache.get_sequence_length(r.sequence_id) for r in survivors) + 1
        return self._graphs.supports(len(survivors), longest)

    def _detach_graph_logits(self, survivors: list[PagedRequest]) -> None:
        """Copies the logits rows of requests that leave the graph batch.

        A graph step's logits are views of a buffer the next replay
        overwrites; requests still decoding get new rows, the others keep a
        copy of their last one.
        """
        if self._graph_step is None:
            return
        staying = {id(r) for r in survivors}
        for request in self._graph_step[0]:
            if id(request) not in staying and request.last_logits is not None:
                request.last_logits = request.last_logits.clone()

    @torch.inference_mode()
    def step(self) -> SchedulerStepOutput:
        """One iteration: the tokens it produced and the requests it finished."""
        if self._closed:
            raise RuntimeError("scheduler is closed")
        if self.config.prefill_chunk_size is not None:
            return self._step_unified_ragged()
        completed = self._admit_pending_requests()
        if not self.active_requests:
            if self.pending_requests and not self.prefilling_requests:
                raise RuntimeError("pending requests cannot be admitted")
            self.completed_requests.extend(completed)
            return SchedulerStepOutput((), tuple(completed))
        next_tokens, token_ids, events = self._sample_active()
        keep = self._retire(token_ids, completed)
        survivors = [self.active_requests[i] for i in keep]
        self.active_requests = survivors
        if survivors:
            try:
                logits = self.model(
                    next_tokens[keep],
                    kv_cache=self.paged_cache,
                    sequence_ids=tuple(r.sequence_id for r in survivors),
                )
                for row, request in enumerate(survivors):
                    request.last_logits = logits[row, -1]
            except Exception as error:
                self._fail_all(survivors, error, completed)
        completed.extend(self._admit_pending_requests())
        self.completed_requests.extend(completed)
        return SchedulerStepOutput(events, tuple(completed))

    def run_until_idle(self) -> tuple[PagedRequest, ...]:
        """Step until every submitted request has finished."""
        finished: list[PagedRequest] = []
        while self.has_work:
            finished.extend(self.step().terminal_requests)
        return tuple(finished)
