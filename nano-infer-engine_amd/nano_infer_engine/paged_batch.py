"""Per-forward device metadata of a ragged paged batch, and the attention core.

The reference engine re-derives block tables, positions and slots inside
every layer from Python tuples (``layers/attention.py:210-261``,
``:363-394``) and moves K/V one token at a time.  Here a forward builds one
:class:`RaggedBatch` (two host-to-device copies) that all layers share:

* ``slot_mapping`` — flat cache slot of every new token (for ``kv_append``),
* ``block_tables`` / ``context_lens`` / ``seq_lens`` / ``cu_seqlens`` — what
  the decode and varlen-prefill kernels read,
* ``positions`` — absolute RoPE position of every new token.

:func:`attention_core` is the per-layer attention core: one fused RoPE +
KV-append launch (``rope_kv_append``), then ``paged_decode`` for requests
with a single new token and ``varlen_prefill`` for the rest.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from nano_infer_engine import _native
from nano_infer_engine.paged_cache import PagedKVCache


#: Decode launches are planned for the longest sequence rounded up to this
#: many tokens (and every decode row at that length), so one plan serves every
#: step until a sequence crosses the next multiple: a captured decode step
#: (``generation.decode_graph``) replays with the same plan, and gives the
#: same results, as the eager step.
DECODE_PLAN_BUCKET = 512


def decode_plan_bound(max_seq_len: int) -> int:
    """Sequence-length bound a decode launch is planned for."""
    return -(-max_seq_len // DECODE_PLAN_BUCKET) * DECODE_PLAN_BUCKET


@dataclass
class RaggedBatch:
    sequence_ids: tuple[str, ...]
    query_lens: tuple[int, ...]
    context_lens: tuple[int, ...]
    num_tokens: int
    # device tensors
    block_tables: torch.Tensor  # (R, W) int32
    context_lens_t: torch.Tensor  # (R,) int32
    seq_lens_t: torch.Tensor  # (R,) int32, context + query
    cu_seqlens: torch.Tensor  # (R + 1,) int64
    slot_mapping: torch.Tensor  # (num_tokens,) int64
    positions: torch.Tensor  # (num_tokens,) int64
    # host-side launch geometry
    decode_from: int  # requests [decode_from, R) have one new token each (a contiguous tail)
    decode_bound: int = 0  # length bound the decode launch is planned for (0: no decode rows)
    # prepared per-layer launches, built on first use (see ``launchers``)
    _launch: dict = field(default_factory=dict, repr=False, compare=False)

    @property
    def num_requests(self) -> int:
        return len(self.sequence_ids)

    @property
    def first_decode_token(self) -> int:
        """Packed row of the first single-token (decode) request."""
        return self.num_tokens - (self.num_requests - self.decode_from)

    @property
    def max_seq_len(self) -> int:
        """Longest sequence after this batch's tokens are appended."""
        return max(c + n for c, n in zip(self.context_lens, self.query_lens))

    def launchers(self, cache: PagedKVCache, q_heads: int, scale: float, rope):
        """(rope + append, prefill or None, decode or None, (cos, sin)) of this batch on ``cache``.

        Built once and reused by every layer: the cache pointers, metadata,
        sin/cos tables, launch plan, workspace and stream are resolved here,
        so a layer's attention costs one C call per kernel family.
        """
        key = (cache.keys.data_ptr(), q_heads, float(scale), id(rope))
        found = self._launch.get(key)
        if found is not None:
            return found
        cos, sin = rope.tables(cache.keys.device, cache.keys.dtype, self.max_seq_len)
        append = _native.PreparedRopeAppend(cache.keys, cache.values, self.positions, self.slot_mapping, cos, sin)
        split = self.decode_from
        prefill = decode = None
        if split > 0:
            seq_lens = [c + n for c, n in zip(self.context_lens[:split], self.query_lens[:split])]
            cu_host = [0]
            for n in self.query_lens[:split]:
                cu_host.append(cu_host[-1] + n)
            prefill = _native.PreparedPrefill(
                cache.keys, cache.values, self.cu_seqlens[: split + 1], self.context_lens_t[:split],
                self.block_tables[:split], self.first_decode_token, max(self.query_lens[:split]), max(seq_lens),
                q_heads, scale, cu_seqlens_host=cu_host, context_lens_host=self.context_lens[:split],
            )
        if split < self.num_requests:
            rows = self.num_requests - split
            decode = _native.PreparedDecode(
                cache.keys, cache.values, self.block_tables[split:], self.seq_lens_t[split:], self.decode_bound,
                rows * self.decode_bound, q_heads, scale,
            )
        found = (append, prefill, decode, (cos, sin))
        self._launch[key] = found
        return found


def build_ragged_batch(
    cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
    query_lens: tuple[int, ...],
    context_lens: tuple[int, ...] | None = None,
) -> RaggedBatch:
    """Metadata for appending ``query_lens[r]`` tokens to each sequence.

    Capacity must already be allocated (``ensure_capacity``).  Context lengths
    default to the cached lengths.
    """
    if context_lens is None:
        context_lens = tuple(cache.get_sequence_length(s) for s in sequence_ids)
    bs = cache.block_size
    for sequence_id, ctx, q in zip(sequence_ids, context_lens, query_lens):
        # every new token must already be backed by a block (same error as a write)
        cache._resolve_position(sequence_id, ctx + q - 1)
    tables = [cache._table(s) for s in sequence_ids]
    num_requests = len(sequence_ids)
    num_tokens = int(sum(query_lens))
    decode_from = num_requests
    while decode_from > 0 and query_lens[decode_from - 1] == 1:
        decode_from -= 1
    decode_bound = 0
    if decode_from < num_requests:
        decode_bound = decode_plan_bound(max(c + 1 for c in context_lens[decode_from:]))
    # rows cover the decode plan's bound, as the decode launch requires
    width = max(1, max(len(t) for t in tables), -(-decode_bound // bs))

    ints = np.zeros(num_requests * width + 2 * num_requests, dtype=np.int32)
    table_view = ints[: num_requests * width].reshape(num_requests, width)
    longs = np.empty(2 * num_tokens + num_requests + 1, dtype=np.int64)
    slots = longs[:num_tokens]
    positions = longs[num_tokens : 2 * num_tokens]
    cu = longs[2 * num_tokens :]
    cu[0] = 0
    cursor = 0
    for r, (table, ctx, q) in enumerate(zip(tables, context_lens, query_lens)):
        table_view[r, : len(table)] = table
        pos = np.arange(ctx, ctx + q, dtype=np.int64)
        positions[cursor : cursor + q] = pos
        slots[cursor : cursor + q] = table_view[r, pos // bs].astype(np.int64) * bs + pos % bs
        cursor += q
        cu[r + 1] = cursor
    ints[num_requests * width : num_requests * width + num_requests] = context_lens
    ints[num_requests * width + num_requests :] = np.asarray(context_lens) + np.asarray(query_lens)

    device = cache.keys.device
    ints_t = torch.from_numpy(ints).to(device, non_blocking=True)
    longs_t = torch.from_numpy(longs).to(device, non_blocking=True)

    return RaggedBatch(
        sequence_ids=tuple(sequence_ids),
        query_lens=tuple(query_lens),
        context_lens=tuple(context_lens),
        num_tokens=num_tokens,
        block_tables=ints_t[: num_requests * width].view(num_requests, width),
        context_lens_t=ints_t[num_requests * width : num_requests * width + num_requests],
        seq_lens_t=ints_t[num_requests * width + num_requests :],
        cu_seqlens=longs_t[2 * num_tokens :],
        slot_mapping=longs_t[:num_tokens],
        positions=longs_t[num_tokens : 2 * num_tokens],
        decode_from=decode_from,
        decode_bound=decode_bound,
    )


def attention_core(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cache: PagedKVCache,
    layer_index: int,
    batch: RaggedBatch,
    scale: float,
    rope,
) -> torch.Tensor:
    """RoPE, append the batch's new K/V to ``layer_index``, and attend.

    q: (num_tokens, Hq, D); k, v: (num_tokens, Hkv, D), not yet rotated.
    Returns the attention context (num_tokens, Hq, D).  q and k are rotated
    at the batch's positions (``layers/attention.py:375-376`` of the
    reference) by the fused RoPE + KV-append kernel, which rotates q in
    place; every new token then attends to its sequence's cached prefix and,
    causally, to the new tokens before it (``layers/attention.py:378-411``).
    """
    append, prefill, decode, rope_tables = batch.launchers(cache, q.shape[1], scale, rope)
    q = _rows(q)
    if prefill is None and decode is not None:
        # decode rows only: RoPE, the append and attention in one launch
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        decode.append_decode(q, _rows(k), _rows(v), layer_index, out, rope_tables=rope_tables)
        return out
    append(q, k, v, layer_index)
    out = torch.empty_like(q)
    split = batch.first_decode_token
    if prefill is not None:
        prefill(q[:split], layer_index, out[:split])
    if decode is not None:
        decode(q[split:], layer_index, out[split:])
    return out


def _rows(t: torch.Tensor) -> torch.Tensor:
    """``t`` if its last dimension is contiguous and its start and other strides
    are 16-byte multiples (a column slice of a fused projection qualifies),
    else an aligned contiguous copy."""
    es = t.element_size()
    if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((st * es) % 16 == 0 for st in t.stride()[:-1]):
        return t
    return t.clone(memory_format=torch.contiguous_format)
