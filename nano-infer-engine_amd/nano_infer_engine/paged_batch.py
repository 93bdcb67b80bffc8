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


#: A captured decode step (``generation.decode_graph``) is captured for the
#: longest sequence rounded up to this many tokens: its tables, grid and
#: workspace cover every step until a sequence crosses the next multiple.
#: Its work items come from the exact plan of each step's lengths, written
#: to device memory with the step's inputs, so a replay computes what the
#: eager step (planned from host lengths) computes.
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
    decode_bound: int = 0  # length bound of a captured decode step's launch (0: no decode rows)
    # a captured step's device plan buffer (``_native.write_decode_plan`` fills
    # it before each replay); None: an eager batch, planned from host lengths
    decode_plan: torch.Tensor | None = None
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
            if self.decode_plan is not None:
                decode = _native.PreparedDecode(
                    cache.keys, cache.values, self.block_tables[split:], self.seq_lens_t[split:], self.decode_bound,
                    rows * self.decode_bound, q_heads, scale, device_plan=self.decode_plan,
                )
            else:
                # the host lengths' plan, as a replay of the step would run it
                # (from bounds when that plan does not fit an item table)
                lens = [c + 1 for c in self.context_lens[split:]]
                keys = cache.keys
                if _native.decode_plan_fits(keys.dtype, q_heads, keys.shape[3], keys.shape[4], keys.shape[2], lens):
                    decode = _native.PreparedDecode(
                        cache.keys, cache.values, self.block_tables[split:], self.seq_lens_t[split:], max(lens),
                        sum(lens), q_heads, scale, seq_lens_host=lens,
                    )
                else:
                    decode = _native.PreparedDecode(
                        cache.keys, cache.values, self.block_tables[split:], self.seq_lens_t[split:],
                        self.decode_bound, rows * self.decode_bound, q_heads, scale,
                    )
        found = (append, prefill, decode, (cos, sin))
        self._launch[key] = found
        return found


class TableMirror:
    """Block-table rows of consecutive steps' batches, maintained in place.

    ``fill`` writes the tables of a batch into an (R, W) staging array that
    it wrote the previous batch into as well.  Row r remembers which
    sequence's table it holds and how many entries of it are written: a
    sequence that kept its row only gets the blocks it gained since (at most
    one per row and step in decoding), a row that changed hands is rewritten
    and its stale tail zeroed.  A change of width or of staging memory
    rewrites everything.  The reference builds these tables anew, as
    tuples, in every layer (``layers/attention.py:258-261``).
    """

    def __init__(self) -> None:
        self._owner: list = []  # per row: the BlockRow written there (None: unknown)
        self._count: list[int] = []  # entries of it written
        self._key: tuple = ()  # (staging address, width) the rows refer to
        self.rewritten = 0  # entries written by the last fill (for tests and measurement)

    def fill(self, view: np.ndarray, rows: list) -> None:
        nrows, width = view.shape
        key = (view.__array_interface__["data"][0], width)
        if key != self._key:
            view[:] = 0
            self._owner, self._count, self._key = [], [], key
        if len(self._owner) < nrows:
            grow = nrows - len(self._owner)
            self._owner.extend([None] * grow)
            self._count.extend([width] * grow)  # unknown content: rewrite the whole row
        written = 0
        for r, row in enumerate(rows):
            n = row.n if row.n < width else width
            k = self._count[r]
            if self._owner[r] is row and k <= n:
                if n > k:
                    view[r, k:n] = row.ids[k:n]
                    written += n - k
            else:
                view[r, :n] = row.ids[:n]
                if k > n:
                    view[r, n:k] = 0
                written += n
                self._owner[r] = row
            self._count[r] = n
        self.rewritten = written


class _Staging:
    """Host staging of a cache's step metadata, reused from step to step:
    int32 [tables (rows x width) | context lens (rows) | sequence lens
    (rows)] and int64 [slots | positions | cu_seqlens].  Pinned when the
    cache is on a GPU, so the two uploads are asynchronous; an event recorded
    after them keeps the next step from rewriting the staging under a copy
    still in flight."""

    def __init__(self, device: torch.device) -> None:
        self.device = device
        self.pinned = device.type == "cuda"
        self.ints = np.zeros(0, dtype=np.int32)
        self.longs = np.zeros(0, dtype=np.int64)
        self._ints_t = self._longs_t = None
        self.rows = self.width = 0
        self.mirror = TableMirror()
        self.uploaded = torch.cuda.Event() if self.pinned else None

    def _buffer(self, size: int, dtype: torch.dtype) -> tuple[torch.Tensor, np.ndarray]:
        t = torch.zeros(size, dtype=dtype, pin_memory=self.pinned)
        return t, t.numpy()

    def layout(self, rows: int, width: int, tokens: int) -> None:
        if self.uploaded is not None:
            self.uploaded.synchronize()
        if rows > self.rows or width != self.width:
            self.rows, self.width = max(rows, self.rows), width
            self._ints_t, self.ints = self._buffer(self.rows * width + 2 * self.rows, torch.int32)
        if 2 * tokens + rows + 1 > self.longs.shape[0]:
            self._longs_t, self.longs = self._buffer(2 * max(2 * tokens + rows + 1, 64), torch.int64)

    def upload(self, tokens: int, rows: int) -> tuple[torch.Tensor, torch.Tensor]:
        n_ints, n_longs = self.rows * self.width + 2 * self.rows, 2 * tokens + rows + 1
        ints = torch.empty(n_ints, dtype=torch.int32, device=self.device)
        longs = torch.empty(n_longs, dtype=torch.int64, device=self.device)
        ints.copy_(self._ints_t[:n_ints], non_blocking=True)
        longs.copy_(self._longs_t[:n_longs], non_blocking=True)
        if self.uploaded is not None:
            self.uploaded.record()
        return ints, longs


def _staging(cache: PagedKVCache) -> _Staging:
    st = getattr(cache, "_step_staging", None)
    if st is None:
        st = _Staging(cache.keys.device)
        cache._step_staging = st
    return st


def build_ragged_batch(
    cache: PagedKVCache,
    sequence_ids: tuple[str, ...],
    query_lens: tuple[int, ...],
    context_lens: tuple[int, ...] | None = None,
) -> RaggedBatch:
    """Metadata for appending ``query_lens[r]`` tokens to each sequence.

    Capacity must already be allocated (``ensure_capacity``).  Context lengths
    default to the cached lengths.  The block tables go through the cache's
    :class:`TableMirror`, so a step rewrites only the table entries that
    changed since the previous one; the rest is vectorised over the batch.
    """
    if context_lens is None:
        context_lens = tuple(cache.get_sequence_length(s) for s in sequence_ids)
    bs = cache.block_size
    rows = [cache._row(s) for s in sequence_ids]
    num_requests = len(sequence_ids)
    ctx = np.asarray(context_lens, dtype=np.int64)
    qlen = np.asarray(query_lens, dtype=np.int64)
    last = ctx + qlen - 1
    capacity = np.fromiter((row.n for row in rows), dtype=np.int64, count=num_requests) * bs
    bad = np.flatnonzero((last >= capacity) | (last < 0))
    if bad.size:
        # every new token must already be backed by a block (same error as a write)
        r = int(bad[0])
        cache._resolve_position(sequence_ids[r], int(last[r]))
    num_tokens = int(qlen.sum())
    decode_from = num_requests
    while decode_from > 0 and query_lens[decode_from - 1] == 1:
        decode_from -= 1
    decode_bound = 0
    if decode_from < num_requests:
        decode_bound = decode_plan_bound(int(ctx[decode_from:].max()) + 1)
    # rows cover the decode plan's bound, as the decode launch requires
    width = max(1, max(row.n for row in rows), -(-decode_bound // bs))

    st = _staging(cache)
    st.layout(num_requests, width, num_tokens)
    table_view = st.ints[: st.rows * width].reshape(st.rows, width)[:num_requests]
    st.mirror.fill(table_view, rows)
    base = st.rows * width
    st.ints[base : base + num_requests] = ctx
    st.ints[base + st.rows : base + st.rows + num_requests] = ctx + qlen
    slots = st.longs[:num_tokens]
    positions = st.longs[num_tokens : 2 * num_tokens]
    cu = st.longs[2 * num_tokens : 2 * num_tokens + num_requests + 1]
    cu[0] = 0
    np.cumsum(qlen, out=cu[1:])
    if num_tokens == num_requests:  # one token per request: vectorised
        positions[:] = ctx
    else:
        positions[:] = np.repeat(ctx - cu[:-1], qlen) + np.arange(num_tokens, dtype=np.int64)
    owner = np.repeat(np.arange(num_requests), qlen)
    slots[:] = table_view[owner, positions // bs].astype(np.int64) * bs + positions % bs

    ints_t, longs_t = st.upload(num_tokens, num_requests)
    tables_t, ctx_t, seq_t = ints_t.split([st.rows * width, st.rows, st.rows])
    slots_t, positions_t, cu_t = longs_t.split([num_tokens, num_tokens, num_requests + 1])
    if st.rows > num_requests:
        ctx_t, seq_t = ctx_t[:num_requests], seq_t[:num_requests]
    return RaggedBatch(
        sequence_ids=tuple(sequence_ids),
        query_lens=tuple(query_lens),
        context_lens=tuple(context_lens),
        num_tokens=num_tokens,
        block_tables=tables_t.view(st.rows, width)[:num_requests],
        context_lens_t=ctx_t,
        seq_lens_t=seq_t,
        cu_seqlens=cu_t,
        slot_mapping=slots_t,
        positions=positions_t,
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
