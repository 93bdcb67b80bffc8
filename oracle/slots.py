"""Closed-form block-table arithmetic (numpy).  Test infrastructure only.

Restates ``paged_cache.py:240-262`` of the reference engine: logical token
position p of a sequence with block table T lives in physical block
T[p // block_size] at offset p % block_size; its flat slot is
T[p // block_size] * block_size + p % block_size.
"""

from __future__ import annotations

import numpy as np


def blocks_needed(token_count: int, block_size: int) -> int:
    """ceil(token_count / block_size)  (``paged_cache.py:92``)."""
    return -(-token_count // block_size)


def resolve(table, position: int, block_size: int) -> tuple[int, int]:
    """(physical block, offset) of one position; IndexError past the table
    (``paged_cache.py:254-262``)."""
    logical, offset = divmod(position, block_size)
    if logical >= len(table):
        raise IndexError("token position exceeds allocated capacity")
    return table[logical], offset


def slot_mapping(tables, context_lens, query_lens, block_size: int) -> np.ndarray:
    """Flat slots of the new tokens of a ragged batch, in packed order."""
    out = []
    for table, ctx, q in zip(tables, context_lens, query_lens):
        for p in range(ctx, ctx + q):
            phys, off = resolve(table, p, block_size)
            out.append(phys * block_size + off)
    return np.asarray(out, dtype=np.int64)


def lifo_allocation_order(num_blocks: int, requests: list[tuple[str, int]]) -> list[list[int]]:
    """Block IDs a LIFO free list seeded (n-1 .. 0) hands out for a sequence
    of ("alloc", n) / ("free", index-of-earlier-alloc) requests
    (``block_allocator.py:15, :35, :60``)."""
    free = list(range(num_blocks - 1, -1, -1))
    grants: list[list[int]] = []
    for kind, arg in requests:
        if kind == "alloc":
            got = [free.pop() for _ in range(arg)]
            grants.append(got)
        else:
            free.extend(reversed(grants[arg]))
            grants.append([])
    return grants
