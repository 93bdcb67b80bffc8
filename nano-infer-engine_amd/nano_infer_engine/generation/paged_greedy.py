"""Synchronous greedy generation of a fixed prompt list through the scheduler.

Observable behaviour follows ``generation/paged_greedy.py:11-91`` of the
reference engine: inputs and capacity are checked before anything is
prefilled (every request must fit the cache on its own; without a batch
limit all of them must fit together), the prompts run FIFO through a
:class:`ContinuousBatchingScheduler` to completion, and the first failed
request's error is raised.
"""

from __future__ import annotations

import torch

from nano_infer_engine.generation.config import GenerationConfig, RaggedGenerationOutput
from nano_infer_engine.generation.paged_prefill import _validate_paged_prefill_inputs
from nano_infer_engine.generation.request import RequestStatus
from nano_infer_engine.generation.scheduler import ContinuousBatchingScheduler, reserved_block_count
from nano_infer_engine.paged_cache import PagedKVCache


@torch.inference_mode()
def paged_greedy_generate(
    model,
    prompts: tuple[torch.Tensor, ...],
    config: GenerationConfig,
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
    *,
    max_batch_size: int | None = None,
) -> RaggedGenerationOutput:
    """Greedy-decode every prompt over a shared paged cache; sequences in input order."""
    if not config.use_cache:
        raise ValueError("paged greedy generation requires config.use_cache=True")
    batch_limited = max_batch_size is not None
    if batch_limited and (isinstance(max_batch_size, bool) or not isinstance(max_batch_size, int)
                          or max_batch_size <= 0):
        raise ValueError("max_batch_size must be a positive integer")
    _validate_paged_prefill_inputs(prompts, paged_cache, sequence_ids)
    free = paged_cache.allocator.free_block_count
    needs = {s: reserved_block_count(p.shape[1], config.max_new_tokens, paged_cache.block_size)
             for p, s in zip(prompts, sequence_ids)}
    too_big = next((s for s, n in needs.items() if n > free), None)
    if too_big is not None:
        raise ValueError(f"request cannot fit in paged cache: {too_big}")
    if not batch_limited and sum(needs.values()) > free:
        raise ValueError("not enough free blocks for paged generation")

    # without a batch limit every request decodes at once and keeps its blocks
    # until the end; with one, a request's blocks are freed at its token limit
    # so the queue behind it can be admitted
    scheduler = ContinuousBatchingScheduler(model, config, paged_cache, max_batch_size or len(prompts),
                                            release_on_token_limit=batch_limited)
    requests = [scheduler.add_request(s, p) for p, s in zip(prompts, sequence_ids)]
    scheduler.run_until_idle()
    for request in requests:
        if request.status is RequestStatus.FAILED:
            raise RuntimeError(f"paged prefill failed: {request.sequence_id}") from request.error
    device = prompts[0].device
    return RaggedGenerationOutput(
        sequences=tuple(r.sequence for r in requests),
        generated_tokens=torch.tensor([r.generated_tokens for r in requests], dtype=torch.long, device=device),
        stopped_by_eos=torch.tensor([r.finished for r in requests], dtype=torch.bool, device=device),
    )
