"""Single-token decode attention straight from paged K/V blocks.

Drop-in for ``layers/paged_attention.py:4-176`` of the reference engine:
same function names, signatures, validation order and messages.  The
attention itself is the gfx950 split-K decode kernel (``nie_paged_decode``)
instead of a Python loop over blocks; block tables are passed as Python
tuples exactly as the reference takes them.
"""

from __future__ import annotations

import torch

from nano_infer_engine import _native


def _is_int(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _validate_common(query, key_cache, value_cache, query_ndim: int) -> None:
    if not isinstance(query, torch.Tensor):
        raise TypeError("query must be a torch.Tensor")
    if not isinstance(key_cache, torch.Tensor) or not isinstance(value_cache, torch.Tensor):
        raise TypeError("key_cache and value_cache must be torch.Tensor objects")
    if query.ndim != query_ndim:
        raise ValueError(f"query must be a {query_ndim}D tensor")
    if key_cache.ndim != 5 or value_cache.ndim != 5:
        raise ValueError("key_cache and value_cache must be 5D tensors")
    if key_cache.shape != value_cache.shape:
        raise ValueError("key_cache and value_cache must have identical shapes")
    if query.dtype != key_cache.dtype or query.dtype != value_cache.dtype:
        raise ValueError("query and K/V caches must have the same dtype")
    if query.device != key_cache.device or query.device != value_cache.device:
        raise ValueError("query and K/V caches must be on the same device")
    if not query.is_floating_point():
        raise ValueError("query and K/V caches must use a floating-point dtype")


def _validate_sequence(
    key_cache: torch.Tensor,
    q_head_num: int,
    head_dim: int,
    block_table: object,
    sequence_length: object,
    layer_index: object,
) -> None:
    """Per-sequence checks of ``paged_attention.py:43-75`` (same order)."""
    if not _is_int(sequence_length):
        raise TypeError("sequence_length must be an integer")
    if sequence_length <= 0:  # type: ignore[operator]
        raise ValueError("sequence_length must be positive")
    if not _is_int(layer_index):
        raise TypeError("layer_index must be an integer")
    if not isinstance(block_table, tuple):
        raise TypeError("block_table must be a tuple")
    num_layers, num_blocks, block_size, kv_head_num, cache_head_dim = key_cache.shape
    if min(key_cache.shape) <= 0:
        raise ValueError("K/V cache dimensions must be positive")
    if not 0 <= layer_index < num_layers:  # type: ignore[operator]
        raise IndexError("layer_index out of range")
    if head_dim != cache_head_dim:
        raise ValueError("query and K/V caches must have the same head dimension")
    if q_head_num % kv_head_num != 0:
        raise ValueError("q_head_num must be divisible by kv_head_num")
    needed = -(-sequence_length // block_size)  # type: ignore[operator]
    if len(block_table) < needed:
        raise ValueError("block_table does not cover sequence_length")
    used = block_table[:needed]
    if any(not _is_int(block_id) for block_id in used):
        raise TypeError("block IDs must be integers")
    if any(block_id < 0 or block_id >= num_blocks for block_id in used):
        raise ValueError("block ID out of range")


def _decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: tuple[tuple[int, ...], ...],
    sequence_lengths: tuple[int, ...],
    layer_index: int,
) -> torch.Tensor:
    block_size = key_cache.shape[2]
    width = max(-(-length // block_size) for length in sequence_lengths)
    rows = [list(table[:width]) + [0] * (width - min(len(table), width)) for table in block_tables]
    device = query.device
    tables = torch.tensor(rows, dtype=torch.int32).to(device, non_blocking=True)
    lengths = torch.tensor(sequence_lengths, dtype=torch.int32).to(device, non_blocking=True)
    head_dim = query.shape[-1]
    return _native.paged_decode(
        query,
        key_cache,
        value_cache,
        layer_index,
        tables,
        lengths,
        max(sequence_lengths),
        sum(sequence_lengths),
        head_dim**-0.5,
    )


def paged_attention_reference(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: tuple[int, ...],
    sequence_length: int,
    layer_index: int,
) -> torch.Tensor:
    """Decode attention of one token (q_head_num, head_dim) over ``sequence_length`` cached tokens.

    key_cache/value_cache: (num_layers, num_blocks, block_size, kv_head_num,
    head_dim).  The current token's K/V must already be cached, so no causal
    mask is needed.  Returns (q_head_num, head_dim) in the query dtype.
    """
    _validate_common(query, key_cache, value_cache, 2)
    q_head_num, head_dim = query.shape
    _validate_sequence(key_cache, q_head_num, head_dim, block_table, sequence_length, layer_index)
    return _decode(query[None], key_cache, value_cache, (block_table,), (sequence_length,), layer_index)[0]


def batched_paged_attention_reference(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: tuple[tuple[int, ...], ...],
    sequence_lengths: tuple[int, ...],
    layer_index: int,
) -> torch.Tensor:
    """Decode attention for a batch (batch, q_head_num, head_dim), one table and length per row."""
    if not isinstance(query, torch.Tensor):
        raise TypeError("query must be a torch.Tensor")
    if query.ndim != 3:
        raise ValueError("query must be a 3D tensor")
    batch_size = query.shape[0]
    if batch_size <= 0:
        raise ValueError("query batch size must be positive")
    if not isinstance(block_tables, tuple):
        raise TypeError("block_tables must be a tuple")
    if not isinstance(sequence_lengths, tuple):
        raise TypeError("sequence_lengths must be a tuple")
    if len(block_tables) != batch_size:
        raise ValueError("block_tables must match the query batch size")
    if len(sequence_lengths) != batch_size:
        raise ValueError("sequence_lengths must match the query batch size")
    if any(not isinstance(table, tuple) for table in block_tables):
        raise TypeError("each block table must be a tuple")
    if any(not _is_int(length) for length in sequence_lengths):
        raise TypeError("sequence lengths must be integers")
    if any(length <= 0 for length in sequence_lengths):
        raise ValueError("sequence lengths must be positive")
    # The reference validates each row as it processes it; validating every
    # row before the single batched launch raises the same errors.
    for row in range(batch_size):
        _validate_common(query[row], key_cache, value_cache, 2)
        q_head_num, head_dim = query.shape[1:]
        _validate_sequence(key_cache, q_head_num, head_dim, block_tables[row], sequence_lengths[row], layer_index)
    return _decode(query, key_cache, value_cache, block_tables, sequence_lengths, layer_index)
