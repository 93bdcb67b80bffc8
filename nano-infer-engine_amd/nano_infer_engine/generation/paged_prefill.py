"""Prompt prefill into the paged cache: whole prompts, or flattened chunks.

Observable behaviour follows ``generation/paged_prefill.py:6-155`` of the
reference engine (its tests match the exceptions and messages):

* :func:`paged_prefill` prefills prompts with one batched model call per
  distinct prompt length, in order of first appearance, and is
  all-or-nothing: if any call fails, every sequence the call list names is
  released before the error propagates;
* :func:`paged_prefill_chunks` packs chunks into one flat token vector with
  ``query_start_loc`` boundaries (the varlen ``cu_seqlens`` layout the
  attention kernels take) and returns each chunk's last-token logits.  For
  this build's ``Llama3_2`` it passes the host-side lengths straight to the
  packed forward and computes logits only for those rows.
"""

from __future__ import annotations

import torch

from nano_infer_engine.models.llama import Llama3_2
from nano_infer_engine.paged_cache import PagedKVCache


def _require(ok: bool, error: type[Exception], message: str) -> None:
    if not ok:
        raise error(message)


def _validate_paged_prefill_inputs(
    prompts: tuple[torch.Tensor, ...],
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
) -> None:
    """Raise on the first malformed input, before the cache is touched."""
    _require(isinstance(paged_cache, PagedKVCache), TypeError, "paged_cache must be a PagedKVCache")
    _require(isinstance(prompts, tuple), TypeError, "prompts must be a tuple")
    _require(isinstance(sequence_ids, tuple), TypeError, "sequence_ids must be a tuple")
    _require(len(prompts) > 0, ValueError, "prompts must not be empty")
    _require(len(prompts) == len(sequence_ids), ValueError, "prompts and sequence_ids must have the same length")
    _require(all(isinstance(s, str) and s for s in sequence_ids), ValueError,
             "sequence IDs must be non-empty strings")
    _require(len(set(sequence_ids)) == len(sequence_ids), ValueError, "sequence IDs must be unique")
    device = paged_cache.keys.device
    for prompt in prompts:
        _require(isinstance(prompt, torch.Tensor), TypeError, "each prompt must be a torch.Tensor")
        _require(prompt.ndim == 2 and prompt.shape[0] == 1, ValueError,
                 "each prompt must have shape (1, prompt_length)")
        _require(prompt.shape[1] > 0, ValueError, "each prompt must contain at least one token")
        _require(prompt.device == device, ValueError, "each prompt must be on the paged cache device")
    taken = next((s for s in sequence_ids if paged_cache.has_sequence(s)), None)
    _require(taken is None, ValueError, f"sequence ID already exists: {taken}")


def _groups_by_length(prompts: tuple[torch.Tensor, ...]) -> list[list[int]]:
    """Prompt indices grouped by prompt length, groups in order of first
    appearance (the order the model calls, and so the block allocations, run)."""
    groups: dict[int, list[int]] = {}
    for index, prompt in enumerate(prompts):
        groups.setdefault(prompt.shape[1], []).append(index)
    return list(groups.values())


@torch.inference_mode()
def paged_prefill(
    model,
    prompts: tuple[torch.Tensor, ...],
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
) -> torch.Tensor:
    """Prefill variable-length prompts; returns (num_prompts, vocab) last-token logits."""
    _validate_paged_prefill_inputs(prompts, paged_cache, sequence_ids)
    _require(sum(paged_cache.blocks_for(p.shape[1]) for p in prompts) <= paged_cache.allocator.free_block_count,
             ValueError, "not enough free blocks")
    last_rows: dict[int, torch.Tensor] = {}
    try:
        for members in _groups_by_length(prompts):
            ids = tuple(sequence_ids[i] for i in members)
            tokens = torch.cat([prompts[i] for i in members], dim=0)
            if len(ids) == 1:
                logits = model(tokens, kv_cache=paged_cache, sequence_id=ids[0])
            else:
                logits = model(tokens, kv_cache=paged_cache, sequence_ids=ids)
            last_rows.update(zip(members, logits[:, -1]))
    except Exception:
        # a batched call may have grown several sequences before failing
        for sequence_id in sequence_ids:
            if paged_cache.has_sequence(sequence_id):
                paged_cache.release(sequence_id)
        raise
    _require(len(last_rows) == len(prompts), RuntimeError, "prefill did not produce logits for every prompt")
    return torch.stack([last_rows[i] for i in range(len(prompts))])


def _is_stock_llama(model) -> bool:
    """This build's Llama3_2, its forward_ragged not replaced on the instance."""
    return isinstance(model, Llama3_2) and "forward_ragged" not in vars(model)


@torch.inference_mode()
def paged_prefill_chunks(
    model,
    chunks: tuple[torch.Tensor, ...],
    paged_cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
) -> torch.Tensor:
    """Append flattened chunks in one forward; returns each chunk's last-token logits."""
    _require(len(chunks) > 0, ValueError, "chunks must not be empty")
    _require(len(chunks) == len(sequence_ids), ValueError, "chunks and sequence_ids must have the same length")
    device = paged_cache.keys.device
    for chunk in chunks:
        _require(isinstance(chunk, torch.Tensor), TypeError, "each chunk must be a torch.Tensor")
        _require(chunk.ndim == 2 and chunk.shape[0] == 1 and chunk.shape[1] > 0, ValueError,
                 "each chunk must have shape (1, chunk_length)")
        _require(chunk.device == device, ValueError, "each chunk must be on the paged cache device")
    _require(len(set(sequence_ids)) == len(sequence_ids), ValueError, "sequence IDs must be unique")

    lengths = tuple(chunk.shape[1] for chunk in chunks)
    bounds = [0]
    for n in lengths:
        bounds.append(bounds[-1] + n)
    flat = torch.cat([chunk.reshape(-1) for chunk in chunks])
    last_rows = torch.tensor(bounds[1:], dtype=torch.long) - 1
    if _is_stock_llama(model):
        # host lengths go straight to the packed forward, and only the rows
        # whose logits are returned reach the final norm and the LM head
        _require(len(sequence_ids) > 0, ValueError, "sequence_ids must be non-empty and unique")
        return model._forward_packed(flat, paged_cache, tuple(sequence_ids), lengths,
                                     last_rows.to(flat.device, non_blocking=True))
    forward_ragged = getattr(model, "forward_ragged", None)
    _require(forward_ragged is not None, TypeError, "model must implement forward_ragged")
    logits = forward_ragged(flat, kv_cache=paged_cache, sequence_ids=sequence_ids,
                            query_start_loc=torch.tensor(bounds, dtype=torch.long).to(flat.device))
    return logits[last_rows.to(logits.device)]
