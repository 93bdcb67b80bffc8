"""Prompt prefill into the paged cache, whole or in flattened chunks.

Behaviour of ``generation/paged_prefill.py:6-155`` of the reference engine:
``paged_prefill`` batches prompts of equal length and is all-or-nothing
(every sequence it touched is released if any call fails);
``paged_prefill_chunks`` packs chunks into one flat token vector with
``query_start_loc`` boundaries (the varlen ``cu_seqlens`` layout) and returns
the logits of each chunk's last token.
"""

from __future__ import annotations

import torch

from nano_infer_engine.models.llama import Llama3_2
from nano_infer_engine.paged_cache import PagedKVCache


def _validate_paged_prefill_inputs(
    prompts: tuple[torch.Tensor, ...],
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
) -> None:
    """Check prefill inputs without touching the cache."""
    if not isinstance(paged_cache, PagedKVCache):
        raise TypeError("paged_cache must be a PagedKVCache")
    if not isinstance(prompts, tuple):
        raise TypeError("prompts must be a tuple")
    if not isinstance(sequence_ids, tuple):
        raise TypeError("sequence_ids must be a tuple")
    if not prompts:
        raise ValueError("prompts must not be empty")
    if len(prompts) != len(sequence_ids):
        raise ValueError("prompts and sequence_ids must have the same length")
    if any(not isinstance(s, str) or not s for s in sequence_ids):
        raise ValueError("sequence IDs must be non-empty strings")
    if len(set(sequence_ids)) != len(sequence_ids):
        raise ValueError("sequence IDs must be unique")
    for prompt in prompts:
        if not isinstance(prompt, torch.Tensor):
            raise TypeError("each prompt must be a torch.Tensor")
        if prompt.ndim != 2 or prompt.shape[0] != 1:
            raise ValueError("each prompt must have shape (1, prompt_length)")
        if prompt.shape[1] <= 0:
            raise ValueError("each prompt must contain at least one token")
        if prompt.device != paged_cache.keys.device:
            raise ValueError("each prompt must be on the paged cache device")
    for sequence_id in sequence_ids:
        if paged_cache.has_sequence(sequence_id):
            raise ValueError(f"sequence ID already exists: {sequence_id}")


@torch.inference_mode()
def paged_prefill(
    model,
    prompts: tuple[torch.Tensor, ...],
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
) -> torch.Tensor:
    """Prefill variable-length prompts; returns (num_prompts, vocab) last-token logits."""
    _validate_paged_prefill_inputs(prompts, paged_cache, sequence_ids)
    needed = sum(paged_cache.blocks_for(p.shape[1]) for p in prompts)
    if needed > paged_cache.allocator.free_block_count:
        raise ValueError("not enough free blocks")

    by_length: dict[int, list[int]] = {}
    for index, prompt in enumerate(prompts):
        by_length.setdefault(prompt.shape[1], []).append(index)

    last_logits: list[torch.Tensor | None] = [None] * len(prompts)
    try:
        for indices in by_length.values():
            batch = torch.cat([prompts[i] for i in indices], dim=0)
            ids = tuple(sequence_ids[i] for i in indices)
            if len(ids) == 1:
                logits = model(batch, kv_cache=paged_cache, sequence_id=ids[0])
            else:
                logits = model(batch, kv_cache=paged_cache, sequence_ids=ids)
            for row, i in enumerate(indices):
                last_logits[i] = logits[row, -1]
    except Exception:
        # A batched call can have touched several sequences before failing.
        for sequence_id in sequence_ids:
            if paged_cache.has_sequence(sequence_id):
                paged_cache.release(sequence_id)
        raise
    if any(v is None for v in last_logits):
        raise RuntimeError("prefill did not produce logits for every prompt")
    return torch.stack(last_logits)  # type: ignore[arg-type]


def _is_stock_llama(model) -> bool:
    """A Llama3_2 whose forward_ragged has not been replaced on the instance."""
    return isinstance(model, Llama3_2) and "forward_ragged" not in vars(model)


@torch.inference_mode()
def paged_prefill_chunks(
    model,
    chunks: tuple[torch.Tensor, ...],
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
) -> torch.Tensor:
    """Append flattened chunks (one forward) and return each chunk's last-token logits."""
    if not chunks:
        raise ValueError("chunks must not be empty")
    if len(chunks) != len(sequence_ids):
        raise ValueError("chunks and sequence_ids must have the same length")
    for chunk in chunks:
        if not isinstance(chunk, torch.Tensor):
            raise TypeError("each chunk must be a torch.Tensor")
        if chunk.ndim != 2 or chunk.shape[0] != 1 or chunk.shape[1] <= 0:
            raise ValueError("each chunk must have shape (1, chunk_length)")
        if chunk.device != paged_cache.keys.device:
            raise ValueError("each chunk must be on the paged cache device")
    if len(set(sequence_ids)) != len(sequence_ids):
        raise ValueError("sequence IDs must be unique")

    flat = torch.cat([chunk[0] for chunk in chunks])
    lengths = [chunk.shape[1] for chunk in chunks]
    starts = [0]
    for n in lengths:
        starts.append(starts[-1] + n)
    last_rows_host = torch.tensor(starts[1:], dtype=torch.long) - 1

    if _is_stock_llama(model):
        # Host-side lengths go straight to the model (no device round trip),
        # and only the rows whose logits are returned reach the LM head.
        if not sequence_ids or len(set(sequence_ids)) != len(sequence_ids):
            raise ValueError("sequence_ids must be non-empty and unique")
        return model._forward_packed(
            flat,
            paged_cache,
            tuple(sequence_ids),
            tuple(lengths),
            last_rows_host.to(flat.device, non_blocking=True),
        )

    try:
        forward_ragged = model.forward_ragged
    except AttributeError:
        raise TypeError("model must implement forward_ragged") from None
    query_start_loc = torch.tensor(starts, dtype=torch.long).to(flat.device)
    logits = forward_ragged(
        flat,
        kv_cache=paged_cache,
        sequence_ids=sequence_ids,
        query_start_loc=query_start_loc,
    )
    return logits[query_start_loc[1:] - 1]
