"""Physical KV-block ID allocator.

Behaviour follows ``block_allocator.py:4-60`` of the reference engine: a LIFO
stack of free IDs that hands out 0, 1, 2, ... on a fresh pool, returns freed
IDs so that the next allocation yields them in the order they were freed, and
validates a whole ``free`` call before it changes any state.  Block tables are
therefore a deterministic function of the request history, which the
bit-exact slot/indexing checks rely on.
"""

from collections.abc import Iterable


def _is_int(value: object) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


class BlockAllocator:
    """Hands out integer IDs of pre-allocated KV blocks."""

    def __init__(self, num_blocks: int) -> None:
        if not _is_int(num_blocks):
            raise TypeError("num_blocks must be an integer")
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        self.num_blocks = num_blocks
        # Top of the stack is the end of the list; seeding it descending makes
        # the first pops return 0, 1, 2, ...
        self._stack: list[int] = list(range(num_blocks))[::-1]
        self._in_use: set[int] = set()

    @property
    def free_block_count(self) -> int:
        return len(self._stack)

    @property
    def allocated_block_count(self) -> int:
        return len(self._in_use)

    def allocate(self, block_count: int = 1) -> list[int]:
        """Pop ``block_count`` IDs (not necessarily contiguous)."""
        if not _is_int(block_count):
            raise TypeError("block_count must be an integer")
        if block_count <= 0:
            raise ValueError("block_count must be positive")
        if block_count > len(self._stack):
            raise ValueError("not enough free blocks")
        taken = self._stack[-block_count:][::-1]
        del self._stack[-block_count:]
        self._in_use.update(taken)
        return taken

    def free(self, block_ids: Iterable[int]) -> None:
        """Return IDs to the pool; the whole call is validated first."""
        ids = list(block_ids)
        for block_id in ids:
            if not _is_int(block_id):
                raise TypeError("block IDs must be integers")
        if len(set(ids)) != len(ids):
            raise ValueError("cannot free the same block more than once")
        for block_id in ids:
            if not 0 <= block_id < self.num_blocks:
                raise ValueError(f"block ID out of range: {block_id}")
            if block_id not in self._in_use:
                raise ValueError(f"block is not allocated: {block_id}")
        self._in_use.difference_update(ids)
        # Push in reverse so the first freed ID is the next one popped.
        self._stack.extend(ids[::-1])
