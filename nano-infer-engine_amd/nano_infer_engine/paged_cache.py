"""Paged KV cache: host-side block tables over one pre-allocated device pool.

Public surface and error behaviour follow ``paged_cache.py:8-374`` of the
reference engine: storage ``keys``/``values`` of shape
(num_layers, num_blocks, block_size, kv_heads, head_dim) allocated once,
per-sequence block tables and lengths kept on the host, the same
validation order and messages.  Data movement (``write``, ``gather``,
``export_sequence``, ``import_sequence``) runs through the gfx950 HIP
library; a cache on a non-GPU device can do all of the bookkeeping but no
data movement.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from nano_infer_engine import _native
from nano_infer_engine.block_allocator import BlockAllocator


def _is_int(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


def _check_sequence_id(sequence_id: object) -> None:
    if not isinstance(sequence_id, str):
        raise TypeError("sequence_id must be a string")
    if not sequence_id:
        raise ValueError("sequence_id must not be empty")


def _check_positive_int(value: object, name: str) -> None:
    if not _is_int(value):
        raise TypeError(f"{name} must be an integer")
    if value <= 0:  # type: ignore[operator]
        raise ValueError(f"{name} must be positive")


class BlockRow:
    """One sequence's block table: physical block IDs in logical order, kept
    in an int32 array with spare capacity, so appending a block is amortised
    O(1) and copying a row into a launch's table is a memcpy, not a
    Python-list conversion.  ``ids[:n]`` are valid; the object lives as long
    as the sequence does (a released and re-created ID gets a new one)."""

    __slots__ = ("ids", "n")

    def __init__(self, blocks: list[int]) -> None:
        self.ids = np.empty(max(8, 2 * len(blocks)), dtype=np.int32)
        self.ids[: len(blocks)] = blocks
        self.n = len(blocks)

    def extend(self, blocks: list[int]) -> None:
        need = self.n + len(blocks)
        if need > self.ids.shape[0]:
            grown = np.empty(max(need, 2 * self.ids.shape[0]), dtype=np.int32)
            grown[: self.n] = self.ids[: self.n]
            self.ids = grown
        self.ids[self.n : need] = blocks
        self.n = need

    def view(self) -> np.ndarray:
        return self.ids[: self.n]


@dataclass(frozen=True)
class PagedKVTransfer:
    """Logical-block snapshot of one sequence, independent of physical IDs.

    ``keys``/``values`` have shape (num_layers, logical_blocks, block_size,
    kv_heads, head_dim); slots past ``sequence_length`` in the last block are
    zero.  Same fields as ``paged_cache.py:8-19`` of the reference.
    """

    sequence_id: str
    sequence_length: int
    block_size: int
    num_layers: int
    kv_head_num: int
    head_dim: int
    keys: torch.Tensor
    values: torch.Tensor


class PagedKVCache:
    """Physical K/V block storage plus per-sequence block tables."""

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        num_layers: int,
        kv_head_num: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str,
    ) -> None:
        _check_positive_int(block_size, "block_size")
        _check_positive_int(num_blocks, "num_blocks")
        _check_positive_int(num_layers, "num_layers")
        _check_positive_int(kv_head_num, "kv_head_num")
        _check_positive_int(head_dim, "head_dim")

        self.block_size = block_size
        self.allocator = BlockAllocator(num_blocks)
        self.num_layers = num_layers
        self.kv_head_num = kv_head_num
        self.head_dim = head_dim

        # sequence ID -> physical block IDs in logical order, and cached length
        self._block_tables: dict[str, BlockRow] = {}
        self._sequence_lengths: dict[str, int] = {}

        shape = (num_layers, num_blocks, block_size, kv_head_num, head_dim)
        self.keys = torch.empty(shape, dtype=dtype, device=device)
        self.values = torch.empty(shape, dtype=dtype, device=device)

    # ------------------------------------------------------------------
    # host bookkeeping
    # ------------------------------------------------------------------
    @property
    def num_blocks(self) -> int:
        return self.allocator.num_blocks

    def blocks_for(self, token_count: int) -> int:
        """Number of blocks that hold ``token_count`` tokens."""
        return -(-token_count // self.block_size)

    def ensure_capacity(self, sequence_id: str, required_tokens: int) -> None:
        """Allocate blocks until ``sequence_id`` can hold ``required_tokens``."""
        _check_sequence_id(sequence_id)
        _check_positive_int(required_tokens, "required_tokens")
        table = self._block_tables.get(sequence_id)
        have = 0 if table is None else table.n
        missing = self.blocks_for(required_tokens) - have
        if missing <= 0:
            return
        # allocate() validates before mutating; the table entry is created
        # only once the allocation succeeded.
        new_blocks = self.allocator.allocate(missing)
        if table is None:
            self._block_tables[sequence_id] = BlockRow(new_blocks)
            self._sequence_lengths[sequence_id] = 0
        else:
            table.extend(new_blocks)

    def get_sequence_length(self, sequence_id: str) -> int:
        _check_sequence_id(sequence_id)
        return self._sequence_lengths.get(sequence_id, 0)

    def advance(self, sequence_id: str, token_count: int) -> None:
        """Grow a sequence's length once every layer has written its tokens."""
        _check_sequence_id(sequence_id)
        _check_positive_int(token_count, "token_count")
        new_length = self._sequence_lengths[sequence_id] + token_count
        self._resolve_position(sequence_id, new_length - 1)  # capacity must exist
        self._sequence_lengths[sequence_id] = new_length

    def get_block_table(self, sequence_id: str) -> tuple[int, ...]:
        """Immutable snapshot of a sequence's block table."""
        _check_sequence_id(sequence_id)
        return tuple(self._block_tables[sequence_id].view().tolist())

    def has_sequence(self, sequence_id: str) -> bool:
        return sequence_id in self._block_tables

    def _table(self, sequence_id: str) -> np.ndarray:
        """Live block table (an int32 view, valid until the sequence grows); KeyError if unknown."""
        return self._block_tables[sequence_id].view()

    def _row(self, sequence_id: str) -> BlockRow:
        """The sequence's table object; KeyError if unknown."""
        return self._block_tables[sequence_id]

    def _lengths(self, sequence_ids) -> list[int]:
        """``get_sequence_length`` of each ID, for callers whose IDs are
        already checked (a decode step's requests)."""
        lengths = self._sequence_lengths
        return [lengths.get(s, 0) for s in sequence_ids]

    def _reserve_next(self, sequence_ids, lengths) -> list[BlockRow]:
        """``ensure_capacity(s, n + 1)`` for each sequence ``s`` of length
        ``n``, for already-checked IDs; returns their table objects.  Only a
        sequence whose last block is full (or that has none) goes through
        ``ensure_capacity`` and the allocator; the others need no change."""
        tables, bs = self._block_tables, self.block_size
        rows = []
        for s, n in zip(sequence_ids, lengths):
            row = tables.get(s)
            if row is None or n >= row.n * bs:
                self.ensure_capacity(s, n + 1)
                row = tables[s]
            rows.append(row)
        return rows

    def _advance_reserved(self, sequence_ids) -> None:
        """``advance(s, 1)`` for sequences whose next position
        ``_reserve_next`` has made room for."""
        lengths = self._sequence_lengths
        for s in sequence_ids:
            lengths[s] += 1

    def _resolve_position(self, sequence_id: str, token_position: int) -> tuple[int, int]:
        """(physical block, offset) of a logical token position."""
        if not _is_int(token_position):
            raise TypeError("token_position must be an integer")
        if token_position < 0:
            raise ValueError("token_position must be non-negative")
        _check_sequence_id(sequence_id)
        row = self._block_tables[sequence_id]
        logical, offset = divmod(token_position, self.block_size)
        if logical >= row.n:
            raise IndexError("token position exceeds allocated capacity")
        return int(row.ids[logical]), offset

    def slots_for(self, sequence_id: str, start_position: int, token_count: int) -> np.ndarray:
        """Flat slots (phys * block_size + offset) of positions start .. start+count-1."""
        table = self._block_tables[sequence_id].view().astype(np.int64)
        positions = np.arange(start_position, start_position + token_count, dtype=np.int64)
        return table[positions // self.block_size] * self.block_size + positions % self.block_size

    def release(self, sequence_id: str) -> None:
        """Return every block of a sequence to the allocator."""
        _check_sequence_id(sequence_id)
        blocks = self._block_tables[sequence_id]
        self.allocator.free(blocks.view().tolist())
        del self._block_tables[sequence_id]
        del self._sequence_lengths[sequence_id]

    # ------------------------------------------------------------------
    # data movement (HIP)
    # ------------------------------------------------------------------
    def _check_layer(self, layer_index: object) -> None:
        if not _is_int(layer_index):
            raise TypeError("layer_index must be an integer")
        if not 0 <= layer_index < self.num_layers:  # type: ignore[operator]
            raise IndexError("layer_index out of range")

    def write(self, layer_index: int, sequence_id: str, start_position: int, keys, values) -> None:
        """Store ``keys``/``values`` (T, kv_heads, head_dim) at positions start..start+T-1."""
        self._check_layer(layer_index)
        _check_sequence_id(sequence_id)
        if not _is_int(start_position):
            raise TypeError("start_position must be an integer")
        if start_position < 0:
            raise ValueError("start_position must be non-negative")
        if not isinstance(keys, torch.Tensor) or not isinstance(values, torch.Tensor):
            raise TypeError("keys and values must be torch.Tensor objects")
        if keys.shape != values.shape:
            raise ValueError("keys and values must have identical shapes")
        if keys.ndim != 3:
            raise ValueError("keys and values must be 3D tensors")
        token_count, kv_heads, head_dim = keys.shape
        if token_count <= 0:
            raise ValueError("keys and values must contain at least one token")
        if kv_heads != self.kv_head_num or head_dim != self.head_dim:
            raise ValueError("keys and values must match the cache KV head count and head dimension")
        if keys.dtype != self.keys.dtype or values.dtype != self.values.dtype:
            raise ValueError("keys and values must match the cache dtype")
        if keys.device != self.keys.device or values.device != self.values.device:
            raise ValueError("keys and values must be on the cache device")
        # The last position must already be backed by a block.
        self._resolve_position(sequence_id, start_position + token_count - 1)
        slots = self.slots_for(sequence_id, start_position, token_count)
        slot_mapping = torch.from_numpy(slots).to(self.keys.device, non_blocking=True)
        _native.kv_append(self.keys, self.values, layer_index, keys, values, slot_mapping)

    def write_slots(self, layer_index: int, keys: torch.Tensor, values: torch.Tensor, slot_mapping: torch.Tensor) -> None:
        """Store token rows at precomputed device slots (one launch for a whole batch)."""
        self._check_layer(layer_index)
        _native.kv_append(self.keys, self.values, layer_index, keys, values, slot_mapping)

    def gather(self, layer_index: int, sequence_id: str, token_count: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Contiguous (token_count, kv_heads, head_dim) K and V of positions 0..token_count-1."""
        self._check_layer(layer_index)
        _check_sequence_id(sequence_id)
        if not _is_int(token_count):
            raise TypeError("token_count must be an integer")
        if token_count <= 0:
            raise ValueError("token_count must be positive")
        self._resolve_position(sequence_id, token_count - 1)
        table = self.table_tensor(sequence_id, self.blocks_for(token_count))
        return _native.kv_gather(self.keys, self.values, layer_index, table, token_count)

    def table_tensor(self, sequence_id: str, blocks: int | None = None) -> torch.Tensor:
        """Device int32 copy of (a prefix of) a sequence's block table."""
        table = self._block_tables[sequence_id].view()
        if blocks is not None:
            table = table[:blocks]
        return torch.from_numpy(table.copy()).to(self.keys.device, non_blocking=True)

    def export_sequence(self, sequence_id: str) -> PagedKVTransfer:
        """Snapshot of a sequence in logical block order (unused tail zeroed)."""
        table = self.get_block_table(sequence_id)
        length = self.get_sequence_length(sequence_id)
        if length <= 0:
            raise ValueError("cannot export an empty sequence")
        count = self.blocks_for(length)
        shape = (self.num_layers, count, self.block_size, self.kv_head_num, self.head_dim)
        keys = torch.empty(shape, dtype=self.keys.dtype, device=self.keys.device)
        values = torch.empty_like(keys)
        blocks = torch.tensor(table[:count], dtype=torch.int32).to(self.keys.device, non_blocking=True)
        _native.kv_copy_blocks(self.keys, self.values, blocks, keys, values, None, count)
        tail = length % self.block_size
        if tail:
            keys[:, -1, tail:].zero_()
            values[:, -1, tail:].zero_()
        return PagedKVTransfer(
            sequence_id=sequence_id,
            sequence_length=length,
            block_size=self.block_size,
            num_layers=self.num_layers,
            kv_head_num=self.kv_head_num,
            head_dim=self.head_dim,
            keys=keys,
            values=values,
        )

    def import_sequence(self, sequence_id: str, transfer: PagedKVTransfer) -> None:
        """Create ``sequence_id`` locally from an exported snapshot."""
        _check_sequence_id(sequence_id)
        if not isinstance(transfer, PagedKVTransfer):
            raise TypeError("transfer must be a PagedKVTransfer")
        if sequence_id in self._block_tables:
            raise ValueError(f"sequence ID already exists: {sequence_id}")
        count = self.blocks_for(transfer.sequence_length)
        expected = (self.num_layers, count, self.block_size, self.kv_head_num, self.head_dim)
        if transfer.sequence_length <= 0:
            raise ValueError("transfer sequence length must be positive")
        if (
            transfer.block_size != self.block_size
            or transfer.num_layers != self.num_layers
            or transfer.kv_head_num != self.kv_head_num
            or transfer.head_dim != self.head_dim
        ):
            raise ValueError("transfer layout does not match the destination cache")
        if transfer.keys.shape != expected:
            raise ValueError("transfer keys have an invalid shape")
        if transfer.values.shape != expected:
            raise ValueError("transfer values have an invalid shape")
        if transfer.keys.dtype != self.keys.dtype:
            raise ValueError("transfer keys must match the cache dtype")
        if transfer.values.dtype != self.values.dtype:
            raise ValueError("transfer values must match the cache dtype")

        self.ensure_capacity(sequence_id, transfer.sequence_length)
        try:
            src_k = transfer.keys.to(self.keys.device).contiguous()
            src_v = transfer.values.to(self.values.device).contiguous()
            blocks = self.table_tensor(sequence_id)
            _native.kv_copy_blocks(src_k, src_v, None, self.keys, self.values, blocks, count)
            self.advance(sequence_id, transfer.sequence_length)
        except Exception:
            self.release(sequence_id)
            raise
