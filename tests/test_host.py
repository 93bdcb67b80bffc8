"""Host-side logic of the paged path (CPU only, no kernel launches).

Restates the checks of the reference's own tests for the block allocator
and the cache bookkeeping (``tests/test_block_allocator.py``,
``tests/test_paged_cache.py:22-200``), plus the ragged-batch metadata that
feeds the kernels, and that data movement refuses to run without a GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_infer_engine import _native
from nano_infer_engine.block_allocator import BlockAllocator
from nano_infer_engine.layers.paged_attention import paged_attention_reference
from nano_infer_engine.paged_batch import build_ragged_batch
from nano_infer_engine.paged_cache import PagedKVCache, PagedKVTransfer
from oracle import slots


# ---------------------------------------------------------------------------
# BlockAllocator (tests/test_block_allocator.py)
# ---------------------------------------------------------------------------
def test_allocator_order_and_counts():
    a = BlockAllocator(4)
    assert (a.free_block_count, a.allocated_block_count) == (4, 0)
    assert a.allocate(2) == [0, 1]
    assert (a.free_block_count, a.allocated_block_count) == (2, 2)


def test_allocator_reuses_freed_blocks_in_free_order():
    a = BlockAllocator(4)
    got = a.allocate(4)
    a.free([got[1], got[3]])
    assert a.allocate(2) == [got[1], got[3]]


def test_allocator_failures_leave_state_unchanged():
    a = BlockAllocator(2)
    with pytest.raises(ValueError, match="not enough free blocks"):
        a.allocate(3)
    assert (a.free_block_count, a.allocated_block_count) == (2, 0)
    b = a.allocate()[0]
    with pytest.raises(ValueError, match="same block more than once"):
        a.free([b, b])
    assert (a.free_block_count, a.allocated_block_count) == (1, 1)
    with pytest.raises(ValueError, match="block is not allocated"):
        a.free([b, 1])
    assert (a.free_block_count, a.allocated_block_count) == (1, 1)
    a.free([b])
    with pytest.raises(ValueError, match="block is not allocated"):
        a.free([b])


@pytest.mark.parametrize("bad,exc,msg", [(0, ValueError, "num_blocks must be positive"),
                                         (-1, ValueError, "num_blocks must be positive"),
                                         (True, TypeError, "num_blocks must be an integer"),
                                         (1.5, TypeError, "num_blocks must be an integer")])
def test_allocator_constructor_validation(bad, exc, msg):
    with pytest.raises(exc, match=msg):
        BlockAllocator(bad)


@pytest.mark.parametrize("bad,exc,msg", [(0, ValueError, "block_count must be positive"),
                                         (True, TypeError, "block_count must be an integer"),
                                         (1.5, TypeError, "block_count must be an integer")])
def test_allocator_allocate_validation(bad, exc, msg):
    with pytest.raises(exc, match=msg):
        BlockAllocator(2).allocate(bad)


@pytest.mark.parametrize("bad,exc,msg", [(-1, ValueError, "block ID out of range"),
                                         (2, ValueError, "block ID out of range"),
                                         (True, TypeError, "block IDs must be integers"),
                                         (1.5, TypeError, "block IDs must be integers")])
def test_allocator_free_validation(bad, exc, msg):
    with pytest.raises(exc, match=msg):
        BlockAllocator(2).free([bad])


# ---------------------------------------------------------------------------
# PagedKVCache bookkeeping (tests/test_paged_cache.py:22-200)
# ---------------------------------------------------------------------------
def _cache(**kw):
    args = dict(num_blocks=4, block_size=4, num_layers=2, kv_head_num=2, head_dim=4, dtype=torch.float32, device="cpu")
    args.update(kw)
    return PagedKVCache(**args)


@pytest.mark.parametrize("tokens,blocks", [(1, 1), (4, 1), (5, 2), (8, 2), (9, 3)])
def test_ensure_capacity_allocates_required_blocks(tokens, blocks):
    c = _cache()
    c.ensure_capacity("request-a", tokens)
    assert len(c.get_block_table("request-a")) == blocks
    assert c.allocator.allocated_block_count == blocks


def test_ensure_capacity_is_incremental_and_tables_are_snapshots():
    c = _cache()
    c.ensure_capacity("request-a", 2)
    first = c.get_block_table("request-a")
    c.ensure_capacity("request-a", 4)
    assert c.get_block_table("request-a") == first
    c.ensure_capacity("request-a", 5)
    assert isinstance(first, tuple) and len(first) == 1
    assert c.get_block_table("request-a")[:1] == first and len(c.get_block_table("request-a")) == 2


def test_lengths_advance_only_within_capacity():
    c = _cache(num_blocks=2)
    assert c.get_sequence_length("request-a") == 0
    c.ensure_capacity("request-a", 4)
    c.advance("request-a", 3)
    c.advance("request-a", 1)
    assert c.get_sequence_length("request-a") == 4
    with pytest.raises(IndexError, match="exceeds allocated capacity"):
        c.advance("request-a", 1)
    assert c.get_sequence_length("request-a") == 4


def test_failed_allocation_creates_no_table():
    c = _cache(num_blocks=2)
    c.ensure_capacity("request-a", 4)
    existing = c.get_block_table("request-a")
    with pytest.raises(ValueError, match="not enough free blocks"):
        c.ensure_capacity("request-b", 8)
    with pytest.raises(KeyError):
        c.get_block_table("request-b")
    assert c.get_block_table("request-a") == existing and c.allocator.free_block_count == 1


def test_tables_of_sequences_are_disjoint_and_release_returns_blocks():
    c = _cache()
    c.ensure_capacity("request-a", 5)
    c.ensure_capacity("request-b", 5)
    a, b = c.get_block_table("request-a"), c.get_block_table("request-b")
    assert set(a).isdisjoint(b)
    c.release("request-a")
    assert c.get_block_table("request-b") == b and c.allocator.allocated_block_count == 2
    with pytest.raises(KeyError, match="request-a"):
        c.release("request-a")
    assert c.allocator.allocate(2) == list(a)


def test_release_keeps_table_when_free_fails(monkeypatch):
    c = _cache(num_blocks=2)
    c.ensure_capacity("request-a", 4)
    table = c.get_block_table("request-a")

    def boom(ids):
        raise RuntimeError("simulated allocator failure")

    monkeypatch.setattr(c.allocator, "free", boom)
    with pytest.raises(RuntimeError, match="simulated allocator failure"):
        c.release("request-a")
    assert c.get_block_table("request-a") == table


@pytest.mark.parametrize("sid,exc,msg", [(None, TypeError, "sequence_id must be a string"),
                                         (1, TypeError, "sequence_id must be a string"),
                                         ("", ValueError, "sequence_id must not be empty")])
def test_sequence_id_validation(sid, exc, msg):
    c = _cache()
    for call in (lambda: c.get_block_table(sid), lambda: c.ensure_capacity(sid, 1),
                 lambda: c.get_sequence_length(sid), lambda: c.release(sid)):
        with pytest.raises(exc, match=msg):
            call()


@pytest.mark.parametrize("n,exc,msg", [(0, ValueError, "required_tokens must be positive"),
                                       (-1, ValueError, "required_tokens must be positive"),
                                       (True, TypeError, "required_tokens must be an integer"),
                                       (1.5, TypeError, "required_tokens must be an integer")])
def test_required_tokens_validation(n, exc, msg):
    with pytest.raises(exc, match=msg):
        _cache().ensure_capacity("request-a", n)


def test_cache_constructor_validation():
    for name in ("num_blocks", "block_size", "num_layers", "kv_head_num", "head_dim"):
        with pytest.raises(ValueError, match=f"{name} must be positive"):
            _cache(**{name: 0})
        with pytest.raises(TypeError, match=f"{name} must be an integer"):
            _cache(**{name: 2.0})


def test_write_validates_before_touching_the_device():
    c = _cache()
    c.ensure_capacity("request-a", 4)
    k = torch.zeros(2, 2, 4)
    with pytest.raises(IndexError, match="layer_index out of range"):
        c.write(2, "request-a", 0, k, k)
    with pytest.raises(ValueError, match="identical shapes"):
        c.write(0, "request-a", 0, k, torch.zeros(1, 2, 4))
    with pytest.raises(ValueError, match="cache dtype"):
        c.write(0, "request-a", 0, k.double(), k.double())
    with pytest.raises(IndexError, match="exceeds allocated capacity"):
        c.write(0, "request-a", 3, k, k)


def test_import_rejects_incompatible_layout_without_allocating():
    c = _cache(num_blocks=2)
    transfer = PagedKVTransfer("request-a", 1, 8, 2, 2, 4, torch.empty(2, 1, 8, 2, 4), torch.empty(2, 1, 8, 2, 4))
    with pytest.raises(ValueError, match="layout does not match"):
        c.import_sequence("request-a", transfer)
    assert c.allocator.allocated_block_count == 0


def test_data_movement_without_gpu_fails_loudly():
    """No CPU fallback: moving K/V on a non-GPU cache raises RuntimeError."""
    c = _cache()
    c.ensure_capacity("request-a", 4)
    k = torch.zeros(2, 2, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        c.write(0, "request-a", 0, k, k)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        c.gather(0, "request-a", 2)
    q = torch.zeros(4, 4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        paged_attention_reference(q, c.keys, c.values, c.get_block_table("request-a"), 2, 0)


# ---------------------------------------------------------------------------
# ragged batch metadata
# ---------------------------------------------------------------------------
def test_ragged_batch_metadata_matches_closed_form():
    c = _cache(num_blocks=16, block_size=4)
    plan = {"p0": (0, 6), "p1": (5, 3), "d0": (9, 1), "d1": (2, 1)}
    for sid, (ctx, n) in plan.items():
        c.ensure_capacity(sid, ctx + n)
        if ctx:
            c.advance(sid, ctx)
    ids = tuple(plan)
    batch = build_ragged_batch(c, ids, tuple(n for _, n in plan.values()))
    tables = [c.get_block_table(s) for s in ids]
    ctx = [plan[s][0] for s in ids]
    qlen = [plan[s][1] for s in ids]
    assert batch.slot_mapping.tolist() == slots.slot_mapping(tables, ctx, qlen, 4).tolist()
    assert batch.cu_seqlens.tolist() == [0, 6, 9, 10, 11]
    assert batch.positions.tolist() == [0, 1, 2, 3, 4, 5, 5, 6, 7, 9, 2]
    assert batch.context_lens_t.tolist() == ctx
    assert batch.seq_lens_t.tolist() == [6, 8, 10, 3]
    assert batch.decode_from == 2
    for r, t in enumerate(tables):
        assert batch.block_tables[r, : len(t)].tolist() == list(t)
    # a token past the allocated capacity is refused before anything is built
    with pytest.raises(IndexError, match="exceeds allocated capacity"):
        build_ragged_batch(c, ("d1",), (3,))


def test_ragged_batch_metadata_over_changing_steps():
    """Steps whose batches grow, shrink, reorder and replace sequences (with
    prefill pieces and decode rows) reuse the cache's staging; every step's
    metadata still equals the closed form of that step alone."""
    rng = np.random.default_rng(7)
    c = _cache(num_blocks=400, block_size=4)
    live: dict[str, int] = {}
    serial = 0
    for step in range(60):
        # retire and admit a few sequences
        for sid in list(live):
            if rng.random() < 0.15:
                if c.has_sequence(sid):
                    c.release(sid)
                del live[sid]
        while len(live) < 6 and rng.random() < 0.8:
            live[f"s{serial}"] = 0
            serial += 1
        ids = list(live)
        rng.shuffle(ids)
        ids = tuple(ids[: int(rng.integers(1, len(ids) + 1))]) if ids else ()
        if not ids:
            continue
        # prefill pieces first, then single-token rows
        qlen = [int(rng.integers(2, 9)) if live[s] < 8 else 1 for s in ids]
        order = sorted(range(len(ids)), key=lambda r: qlen[r] == 1)
        ids = tuple(ids[r] for r in order)
        qlen = tuple(qlen[r] for r in order)
        for s, n in zip(ids, qlen):
            c.ensure_capacity(s, live[s] + n)
        batch = build_ragged_batch(c, ids, qlen)
        ctx = [live[s] for s in ids]
        tables = [c.get_block_table(s) for s in ids]
        assert batch.slot_mapping.tolist() == slots.slot_mapping(tables, ctx, list(qlen), 4).tolist()
        assert batch.positions.tolist() == [p for cx, n in zip(ctx, qlen) for p in range(cx, cx + n)]
        assert batch.cu_seqlens.tolist() == np.concatenate([[0], np.cumsum(qlen)]).tolist()
        assert batch.context_lens_t.tolist() == ctx
        assert batch.seq_lens_t.tolist() == [cx + n for cx, n in zip(ctx, qlen)]
        width = batch.block_tables.shape[1]
        for r, t in enumerate(tables):
            assert batch.block_tables[r].tolist() == list(t[:width]) + [0] * (width - min(len(t), width)), (step, r)
        for s, n in zip(ids, qlen):
            c.advance(s, n)
            live[s] += n


def test_table_mirror_rewrites_only_what_changed():
    from nano_infer_engine.paged_batch import TableMirror

    c = _cache(num_blocks=64, block_size=4)
    for sid, n in (("a", 9), ("b", 4), ("c", 13)):
        c.ensure_capacity(sid, n)
    view = np.full((3, 8), -1, dtype=np.int32)
    m = TableMirror()
    rows = [c._row(s) for s in ("a", "b", "c")]
    m.fill(view, rows)
    assert m.rewritten == 3 + 1 + 4
    assert view[0, :3].tolist() == list(c.get_block_table("a")) and view[0, 3:].tolist() == [0] * 5
    m.fill(view, rows)  # nothing changed
    assert m.rewritten == 0
    c.ensure_capacity("b", 5)  # b gains one block
    m.fill(view, rows)
    assert m.rewritten == 1 and view[1, :2].tolist() == list(c.get_block_table("b"))
    # another sequence takes row 2: the row is rewritten and its stale tail zeroed
    c.ensure_capacity("d", 2)
    m.fill(view, [rows[0], rows[1], c._row("d")])
    assert m.rewritten == 1
    assert view[2].tolist() == list(c.get_block_table("d")) + [0] * 7


# ---------------------------------------------------------------------------
# the C ABI library (loads and exports; no compute without a GPU)
# ---------------------------------------------------------------------------
def _header_symbols():
    import os
    import re

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "nie_paged.h")
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nie_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = _native.load_library()
    declared = _header_symbols()
    assert declared == sorted(_native.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.nie_version().decode().startswith("nie_paged")


@pytest.fixture
def fast_rounding():
    """The one-pass (online softmax) rounding mode for the test's duration."""
    _native.set_attention_rounding("fast")
    try:
        yield
    finally:
        _native.set_attention_rounding("reference")


def test_attention_rounding_mode_switch():
    assert _native.attention_rounding() == "reference"  # the default: the reference's rounding point
    lib = _native.load_library()
    try:
        _native.set_attention_rounding("fast")
        assert _native.attention_rounding() == "fast" and lib.nie_attention_rounding() == _native.NIE_ROUND_FAST
    finally:
        _native.set_attention_rounding("reference")
    assert lib.nie_attention_rounding() == _native.NIE_ROUND_REFERENCE
    assert lib.nie_set_attention_rounding(7) == -1 and b"NIE_ROUND" in lib.nie_last_error()
    with pytest.raises(ValueError, match="attention rounding"):
        _native.set_attention_rounding("exact")


def test_library_workspace_queries(fast_rounding):
    lib = _native.load_library()
    # every workspace starts with the 256 KiB control region
    ctl = _native.workspace_control_bytes()
    assert ctl == 256 * 1024
    # decode partials: items * q_heads * (head_dim + 2) floats, items bounded by the split count
    small = lib.nie_paged_decode_workspace_bytes(1, 4, 32, 8, 64, 16, 500, 710, None) - ctl
    assert small > 0 and small % (32 * 66 * 4) == 0
    big = lib.nie_paged_decode_workspace_bytes(1, 16, 32, 8, 64, 16, 29600, 16 * 29600, None) - ctl
    assert big >= small
    # at most 128 tiles of 16 keys per split (the block-table window): at least 16 * ceil(1850 / 128) items
    assert big >= 16 * 15 * 32 * 66 * 4
    # the reference rounding adds a bf16 score for every key slot of every query head: planned on the
    # device, (tiles + 128 per sequence) * 16 slots; fp32 calls do not round probabilities (no scores)
    _native.set_attention_rounding("reference")
    ref = lib.nie_paged_decode_workspace_bytes(1, 4, 32, 8, 64, 16, 500, 710, None)
    assert ref == ctl + -(-small // 256) * 256 + (-(-710 // 16) + 4 * 128) * 16 * 32 * 2
    assert (lib.nie_paged_decode_workspace_bytes(0, 4, 32, 8, 64, 16, 500, 710, None)
            == lib.nie_paged_decode_workspace_bytes(0, 4, 32, 8, 64, 16, 500, 710, None))
    _native.set_attention_rounding("fast")
    assert lib.nie_paged_decode_workspace_bytes(0, 4, 32, 8, 64, 16, 500, 710, None) > 0
    assert lib.nie_paged_decode_workspace_bytes(1, 0, 32, 8, 64, 16, 1, 1, None) == 0
    assert lib.nie_paged_decode_workspace_bytes(7, 4, 32, 8, 64, 16, 500, 710, None) == 0  # bad dtype
    # head_dim 96 and GQA group 3 run on the generic kernel, which needs no workspace
    assert lib.nie_paged_decode_workspace_bytes(1, 4, 32, 8, 96, 16, 500, 710, None) == 0
    assert lib.nie_paged_decode_workspace_bytes(1, 4, 24, 8, 64, 16, 500, 710, None) == 0
    assert lib.nie_varlen_prefill_workspace_bytes(4, 512, 128, 4128, 32, 8, 3, None, None) == 0
    assert lib.nie_paged_decode_workspace_bytes(1, 4, 32, 8, 512, 16, 500, 710, None) == 0  # beyond 256
    assert _native.tuned_attention(32, 8, 64) and not _native.tuned_attention(32, 8, 3)
    assert not _native.tuned_attention(24, 8, 64)
    # prefill, planned from bounds
    assert lib.nie_varlen_prefill_workspace_bytes(4, 512, 128, 4128, 32, 8, 64, None, None) > 0


def test_library_decode_plan_from_host_lengths():
    """With host lengths the decode plan is exact: 16 sequences of 29,600
    tokens (1,850 tiles each) fill the 256 resident workgroups with 16 splits
    of 116 tiles (the bound-based plan uses 240), and lengths that do not
    match max / total are rejected."""
    lib = _native.load_library()

    def query(lens, mx, total):
        lens = np.asarray(lens, dtype=np.int32)
        return lib.nie_paged_decode_workspace_bytes(1, len(lens), 32, 8, 64, 16, mx, total, lens.ctypes.data)

    # reference rounding: the control region, the partials, then a bf16 score per key slot (256 items x
    # 116 tiles x 16) and head
    ctl = _native.workspace_control_bytes()
    assert query([29600] * 16, 29600, 16 * 29600) == ctl + 256 * 32 * 66 * 4 + 256 * 116 * 16 * 32 * 2
    _native.set_attention_rounding("fast")
    try:
        assert query([29600] * 16, 29600, 16 * 29600) == ctl + 256 * 32 * 66 * 4
        # the bound-based plan (124-tile splits: 240 items) sizes for an upper bound on its items
        assert (lib.nie_paged_decode_workspace_bytes(1, 16, 32, 8, 64, 16, 29600, 16 * 29600, None)
                >= ctl + 240 * 32 * 66 * 4)
    finally:
        _native.set_attention_rounding("reference")
    assert query([29600] * 16, 29600, 16 * 29600 - 1) == 0  # sum does not match
    assert query([29600] * 15 + [0], 29600, 15 * 29600) == 0  # a length below 1


def test_library_prefill_plan_from_host_lengths():
    """With host copies of the lengths the prefill plan uses the exact work:
    split partials exist only when some query tile's keys are split, are a
    whole number of (items x kv_heads x 128 rows x (64 + 4) floats: the
    partial O rows and two (max, sum) slots per row), and lengths that do
    not fit the call's sizes are rejected."""
    lib = _native.load_library()

    def query(cu, ctx, total, max_q, max_s):
        cu = np.asarray(cu, dtype=np.int64)
        ctx = np.asarray(ctx, dtype=np.int32)
        return lib.nie_varlen_prefill_workspace_bytes(len(ctx), total, max_q, max_s, 32, 8, 64,
                                                      cu.ctypes.data, ctx.ctypes.data)

    # four 128-token chunks on empty contexts: at most 8 key tiles per query tile, never split, so the
    # one-pass rounding needs no workspace; the reference rounding keeps every item's (max, sum) slots
    # in the same layout (16 items here: 4 query tiles of 32 tokens per chunk), after the control region
    ctl = _native.workspace_control_bytes()
    assert query([0, 128, 256, 384, 512], [0, 0, 0, 0], 512, 128, 128) == ctl + 16 * 8 * 128 * 68 * 4
    _native.set_attention_rounding("fast")
    try:
        assert query([0, 128, 256, 384, 512], [0, 0, 0, 0], 512, 128, 128) == 0
    finally:
        _native.set_attention_rounding("reference")
    # the mixed step's chunks (contexts 0, 384, 1024, 4000): the long context is split
    mixed = query([0, 128, 256, 384, 512], [0, 384, 1024, 4000], 512, 128, 4128) - ctl
    assert mixed > 0 and mixed % (8 * 128 * 68 * 4) == 0
    # lengths that do not match the sizes of the call
    assert query([0, 128, 256, 384, 500], [0, 384, 1024, 4000], 512, 128, 4128) == 0
    assert query([0, 128, 256, 384, 512], [0, 384, 1024, 4001], 512, 128, 4128) == 0


def test_decoder_kernel_support_checks():
    """The shapes the RMSNorm / SiLU-product kernels take (16-byte rows, at most
    1024 vectors per norm row), decided on the host before any launch."""
    bf = torch.empty((16, 2048), dtype=torch.bfloat16)
    assert _native.rms_norm_supported(bf) and _native.silu_mul_supported(bf)
    assert _native.rms_norm_supported(torch.empty((3, 8192), dtype=torch.bfloat16))
    assert not _native.rms_norm_supported(torch.empty((3, 8200), dtype=torch.bfloat16))  # > 1024 vectors
    assert not _native.rms_norm_supported(torch.empty((3, 12), dtype=torch.bfloat16))  # not whole vectors
    assert _native.silu_mul_supported(torch.empty((3, 16384), dtype=torch.float32))
    assert not _native.silu_mul_supported(torch.empty((3, 6), dtype=torch.float32))
    assert not _native.rms_norm_supported(torch.empty((3, 64), dtype=torch.float16))


def test_linear_rows_support_checks():
    """The projections nie_linear_rows takes (bf16 GPU tensors, at most 16 rows,
    in-features a multiple of 2048, out-features a multiple of 16); CPU tensors
    and other shapes stay with torch's GEMM."""
    x = torch.empty((16, 2048), dtype=torch.bfloat16)
    w = torch.empty((3072, 2048), dtype=torch.bfloat16)
    assert not _native.linear_rows_supported(x, w)  # CPU tensors
    meta = torch.device("meta")
    xm, wm = x.to(meta), w.to(meta)
    assert not _native.linear_rows_supported(xm, wm)  # not a GPU device
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        _native.linear_rows(x, w)


def test_kv_copy_blocks_validates_shapes_before_touching_the_device():
    """The block-copy kernel indexes V with K's geometry and a packed side
    with `count` blocks per layer, so mismatched tensors are refused on the
    host (ValueError) before any device check or launch."""
    pool = torch.zeros((2, 10, 4, 2, 8))
    staged = torch.zeros((2, 3, 4, 2, 8))
    blocks = torch.tensor([1, 5, 7], dtype=torch.int32)
    with pytest.raises(ValueError, match="shape of their K"):
        _native.kv_copy_blocks(pool, torch.zeros((2, 9, 4, 2, 8)), blocks, staged, staged.clone(), None, 3)
    with pytest.raises(ValueError, match="shape of their K"):
        _native.kv_copy_blocks(pool, pool.clone(), blocks, staged, torch.zeros((2, 4, 4, 2, 8)), None, 3)
    with pytest.raises(ValueError, match="packed destination"):
        _native.kv_copy_blocks(pool, pool.clone(), blocks, staged, staged.clone(), None, 2)
    with pytest.raises(ValueError, match="packed source"):
        _native.kv_copy_blocks(staged, staged.clone(), None, pool, pool.clone(), blocks, 2)
    with pytest.raises(ValueError, match="`count` entries"):
        _native.kv_copy_blocks(pool, pool.clone(), blocks[:2], staged, staged.clone(), None, 3)
    # consistent shapes pass validation and stop at the device check
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        _native.kv_copy_blocks(pool, pool.clone(), blocks, staged, staged.clone(), None, 3)


@pytest.mark.parametrize(
    "rows,n,k,silu,built",
    [(16, 3072, 2048, False, True), (1, 16384, 2048, True, True), (16, 2048, 8192, False, True),
     (16, 8192, 4096, True, True),
     # in-feature sizes the library has no instantiation for stay with torch's GEMM
     (16, 4096, 14336, False, False), (16, 2048, 6144, False, False), (16, 16384, 8192, True, False),
     (17, 3072, 2048, False, False), (16, 3080, 2048, False, False), (16, 48, 2048, True, False)],
)
def test_linear_rows_predicate_matches_the_built_kernels(rows, n, k, silu, built):
    """The host predicate admits exactly the shapes the C entry point accepts
    (its check_linear: k 2048 / 4096, or 8192 without the SwiGLU epilogue), so
    every other projection falls back to torch's GEMM instead of raising."""
    assert _native.linear_rows_shape_built(rows, n, k, silu) is built


def test_rope_table_validation():
    """RoPE tables for the fused decode: (rows, head_dim / 2), the query dtype,
    contiguous, the same shape; None means no rotation."""
    cpu = torch.device("cpu")
    assert _native._check_rope_tables(None, 64, torch.bfloat16, cpu) == (None, None, 0)
    cos = torch.zeros((10, 32), dtype=torch.bfloat16)
    sin = torch.zeros((10, 32), dtype=torch.bfloat16)
    _, _, rows = _native._check_rope_tables((cos, sin), 64, torch.bfloat16, cpu)
    assert rows == 10
    for bad in [(cos, sin[:5]), (cos.float(), sin), (cos[:, :16], sin[:, :16]), (cos.t(), sin.t())]:
        with pytest.raises(ValueError):
            _native._check_rope_tables(bad, 64, torch.bfloat16, cpu)


def test_request_joins_generated_tokens_when_read():
    """PagedRequest.sequence: the prompt followed by the appended tokens, joined
    once when read; assigning replaces it."""
    from nano_infer_engine.generation.request import PagedRequest

    prompt = torch.tensor([[5, 6, 7]])
    r = PagedRequest("s", prompt)
    assert r.sequence is prompt
    step = torch.tensor([[1], [2]])
    r.append_token(step[1:2])
    r.append_token(torch.tensor([[9]]))
    assert r.sequence.tolist() == [[5, 6, 7, 2, 9]]
    assert r.sequence.tolist() == [[5, 6, 7, 2, 9]]  # joined once, stable
    r.append_token(torch.tensor([[4]]))
    assert r.sequence.tolist() == [[5, 6, 7, 2, 9, 4]]
    r._append_row(step, 0)  # a step's row, sliced when the sequence is read
    r.append_token(torch.tensor([[8]]))
    r._append_row(step, 1)
    assert r.sequence.tolist() == [[5, 6, 7, 2, 9, 4, 1, 8, 2]]
    r.sequence = prompt
    assert r.sequence is prompt


def test_rms_norm_forward_add_on_cpu_is_add_then_norm():
    """RmsNorm.forward_add: (x + residual, norm(x + residual)), the reference's
    residual add then norm (layers/decoder.py:50-51), on the CPU path."""
    from nano_infer_engine.layers.rms_norm import RmsNorm

    torch.manual_seed(0)
    norm = RmsNorm(64, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(64))
    x, r = torch.randn(5, 64).bfloat16(), torch.randn(5, 64).bfloat16()
    norm = norm.bfloat16()
    h, n = norm.forward_add(x, r)
    assert torch.equal(h, x + r)
    assert torch.equal(n, norm(x + r))


def test_unsummed_residual_chain_equals_summed_on_cpu():
    """Decoder blocks passing their output as an unsummed (ffn_out, h) pair to
    the next norm give the same values as summing first (CPU path)."""
    from nano_infer_engine.layers.decoder import Llama3Decoder

    torch.manual_seed(1)
    blocks = [Llama3Decoder(1e-5, 4, 2, 64, 128) for _ in range(2)]

    def fake_attention(normed, *args):  # deterministic stand-in for the paged attention
        return torch.tanh(normed)

    for b in blocks:
        b.attn.forward_tokens = fake_attention
    x = torch.randn(3, 64)
    summed = x
    for b in blocks:
        summed = b.forward_tokens(summed, None, 0, None)
    pair = x
    for b in blocks:
        pair = b.forward_tokens_unsummed(pair, None, 0, None)
    assert torch.equal(summed, pair[0] + pair[1])


def test_library_rejects_bad_decoder_and_fused_arguments():
    """The new entry points validate before any launch: unsupported dtype or
    row length, null pointers and misaligned rows return an error status (and
    an empty batch returns 0), so no kernel sees a bad shape."""
    lib = _native.load_library()
    buf = torch.zeros(4096, dtype=torch.uint8)
    p = buf.data_ptr() + (-buf.data_ptr()) % 16  # a 16-byte aligned host address (never dereferenced)
    # nie_rms_norm(dtype, x, x_stride, res, res_stride, sum, sum_stride, w, out, out_stride, rows, cols, eps, stream)
    assert lib.nie_rms_norm(7, p, 64, None, 0, None, 0, None, p, 64, 4, 64, 1e-5, None) < 0  # dtype
    assert lib.nie_rms_norm(1, p, 64, None, 0, None, 0, None, p, 64, 4, 12, 1e-5, None) < 0  # 12 columns
    assert lib.nie_rms_norm(1, p, 9000, None, 0, None, 0, None, p, 9000, 4, 9000, 1e-5, None) < 0  # too long
    assert lib.nie_rms_norm(1, None, 64, None, 0, None, 0, None, p, 64, 4, 64, 1e-5, None) < 0  # null x
    assert lib.nie_rms_norm(1, p, 64, p, 64, None, 0, None, p, 64, 4, 64, 1e-5, None) < 0  # residual, no sum
    assert lib.nie_rms_norm(1, p + 2, 64, None, 0, None, 0, None, p, 64, 4, 64, 1e-5, None) < 0  # misaligned
    assert lib.nie_rms_norm(1, p, 32, None, 0, None, 0, None, p, 64, 4, 64, 1e-5, None) < 0  # stride < cols
    assert lib.nie_rms_norm(1, p, 64, None, 0, None, 0, None, p, 64, 0, 64, 1e-5, None) == 0  # no rows
    # nie_silu_mul(dtype, gate, gate_stride, up, up_stride, out, out_stride, rows, cols, stream)
    assert lib.nie_silu_mul(1, p, 64, p, 64, p, 64, 4, 12, None) < 0  # 12 columns
    assert lib.nie_silu_mul(1, None, 64, p, 64, p, 64, 4, 64, None) < 0  # null gate
    assert lib.nie_silu_mul(1, p + 2, 64, p, 64, p, 64, 4, 64, None) < 0  # misaligned
    assert lib.nie_silu_mul(1, p, 64, p, 64, p, 64, 0, 64, None) == 0  # no rows
    # nie_linear_rows(dtype, x, x_stride, rows, w, n, k, epilogue, y, y_stride, stream)
    assert lib.nie_linear_rows(0, p, 2048, 4, p, 64, 2048, 0, p, 64, None) == -2  # fp32 is not built
    assert lib.nie_linear_rows(1, p, 2048, 17, p, 64, 2048, 0, p, 64, None) == -2  # 17 rows
    assert lib.nie_linear_rows(1, p, 2048, 0, p, 64, 2048, 0, p, 64, None) == -2  # no rows
    assert lib.nie_linear_rows(1, p, 1024, 4, p, 64, 1024, 0, p, 64, None) == -2  # k not a multiple of 2048
    assert lib.nie_linear_rows(1, p, 2048, 4, p, 40, 2048, 0, p, 40, None) == -2  # n not a multiple of 16
    assert lib.nie_linear_rows(1, p, 2048, 4, p, 64, 2048, 2, p, 64, None) == -1  # unknown epilogue
    assert lib.nie_linear_rows(1, None, 2048, 4, p, 64, 2048, 0, p, 64, None) == -1  # null x
    assert lib.nie_linear_rows(1, p + 2, 2048, 4, p, 64, 2048, 0, p, 64, None) == -1  # misaligned x
    assert lib.nie_linear_rows(1, p, 2052, 4, p, 64, 2048, 0, p, 64, None) == -1  # x rows misaligned
    assert lib.nie_linear_rows(1, p, 1024, 4, p, 64, 2048, 0, p, 64, None) == -1  # x stride < k
    assert lib.nie_linear_rows(1, p, 2048, 4, p, 64, 2048, 0, p, 32, None) == -1  # y stride < n
    assert b"linear_rows" in lib.nie_last_error()
    # nie_rms_norm_linear_rows(dtype, x, xs, res, rs, sum, ss, norm_w, eps, rows, w, n, k, epi, y, ys, stream)
    assert lib.nie_rms_norm_linear_rows(1, p, 4096, None, 0, None, 0, p, 1e-5, 4, p, 64, 4096, 0, p, 64, None) == -2
    assert lib.nie_rms_norm_linear_rows(1, p, 2048, None, 0, None, 0, None, 1e-5, 4, p, 64, 2048, 0, p, 64,
                                        None) == -1  # no norm weight
    assert lib.nie_rms_norm_linear_rows(1, p, 2048, None, 0, p, 2048, p, 1e-5, 4, p, 64, 2048, 0, p, 64,
                                        None) == -1  # sum_out without a residual
    assert lib.nie_rms_norm_linear_rows(1, p, 2048, p, 1024, None, 0, p, 1e-5, 4, p, 64, 2048, 0, p, 64,
                                        None) == -1  # residual rows shorter than k
    assert lib.nie_rms_norm_linear_rows(1, p, 2048, None, 0, None, 0, p, -1.0, 4, p, 64, 2048, 0, p, 64,
                                        None) == -1  # negative eps
    assert lib.nie_rms_norm_linear_rows(1, p, 2048, None, 0, None, 0, p + 2, 1e-5, 4, p, 64, 2048, 0, p, 64,
                                        None) == -1  # misaligned norm weight
    assert b"rms_norm_linear_rows" in lib.nie_last_error()
    # nie_argmax_rows_split(dtype, logits, rows, cols, row_stride, out, ws, ws_bytes, stream)
    need = lib.nie_argmax_rows_workspace_bytes(16, 128256)
    assert need == 16 * 16 * 16  # 16 pieces of 8192 columns per row, 16 bytes per pair
    assert lib.nie_argmax_rows_workspace_bytes(0, 100) == 0
    assert lib.nie_argmax_rows_split(1, p, 16, 128256, 128256, p, p, need - 16, None) == -1  # workspace too small
    assert lib.nie_argmax_rows_split(1, p, 16, 128256, 128256, p, p + 8, need, None) == -1  # misaligned
    assert lib.nie_argmax_rows_split(1, p, 16, 128256, 100, p, p, need, None) == -1  # stride < cols
    assert lib.nie_argmax_rows_split(1, p, 16, 128256, 128256, p, None, need, None) == -1  # no workspace
    assert lib.nie_argmax_rows_split(1, p, 0, 128256, 128256, p, p, need, None) == 0  # no rows
    # nie_paged_decode_append with a batch but no new rows, or one RoPE table only
    args = dict(q=p, k_cache=p, v_cache=p, tables=p, lens=p, out=p)
    base = [1, args["q"], 32 * 64, 64]
    rest = [args["k_cache"], args["v_cache"], 1, 0, 4, 16, 32, 8, 64, args["tables"], 4, args["lens"], 2, 40, 60,
            0.125, args["out"], 32 * 64, 64, p, 1 << 20, None, None]
    assert lib.nie_paged_decode_append(*base, None, 512, p, 512, None, None, 0, *rest) < 0  # no new keys
    assert lib.nie_paged_decode_append(*base, p, 512, p, 512, p, None, 4, *rest) < 0  # one table
    assert b"RoPE" in lib.nie_last_error()


def test_lean_weight_key_follows_parameters_and_tolerates_weightless_norms():
    """The key that keeps a block's cached lean weights valid changes when a
    weight is modified in place, replaced, or given a bias, or when a norm's
    eps changes; a block with a weightless norm is simply not taken (on the
    CPU no block is: the lean path needs the HIP kernels)."""
    from torch import nn

    from nano_infer_engine.layers.decoder import Llama3Decoder
    from nano_infer_engine.layers.rms_norm import RmsNorm

    d = Llama3Decoder(1e-5, 4, 2, 64, 128)
    x = torch.zeros(3, 64)
    keys = [d._lean_key(x)]
    assert d._lean_key(x) == keys[0]
    with torch.no_grad():
        d.attn.o_proj.weight.mul_(2)
    keys.append(d._lean_key(x))
    d.ffn.up_proj.weight = nn.Parameter(d.ffn.up_proj.weight.detach().clone())
    keys.append(d._lean_key(x))
    d.attn.k_proj.bias = nn.Parameter(torch.zeros(d.attn.k_proj.weight.shape[0]))
    keys.append(d._lean_key(x))
    d.post_norm.eps = 1e-6
    keys.append(d._lean_key(x))
    keys.append(d._lean_key(x.to(torch.bfloat16)))
    assert len(set(keys)) == len(keys)
    d.pre_norm = RmsNorm(64, elementwise_affine=False)
    assert d.lean_weights(x) is False


def test_decode_step_bookkeeping_fast_path_matches_public_methods():
    """The graph runner's per-step bookkeeping (_lengths, _reserve_next,
    _advance_reserved) leaves the cache as get_sequence_length,
    ensure_capacity(s, n + 1) and advance(s, 1) do: the same lengths, block
    tables and allocator order, over steps that cross block boundaries and
    with sequences that start empty."""
    public = PagedKVCache(64, 4, 1, 1, 8, torch.float32, torch.device("cpu"))
    fast = PagedKVCache(64, 4, 1, 1, 8, torch.float32, torch.device("cpu"))
    for c in (public, fast):
        c.ensure_capacity("a", 6)
        c.advance("a", 6)
        c.ensure_capacity("b", 1)
        c.advance("b", 1)
    ids = ["a", "b"]
    for step in range(40):
        if step == 7:
            ids = ids + ["c"]  # a sequence with no table yet
        lengths = [public.get_sequence_length(s) for s in ids]
        for s, n in zip(ids, lengths):
            public.ensure_capacity(s, n + 1)
        for s in ids:
            public.advance(s, 1)
        got = fast._lengths(ids)
        assert got == lengths
        rows = fast._reserve_next(ids, got)
        assert [r.view().tolist() for r in rows] == [list(public.get_block_table(s)) for s in ids]
        fast._advance_reserved(ids)
        for s in ids:
            assert fast.get_sequence_length(s) == public.get_sequence_length(s)
            assert fast.get_block_table(s) == public.get_block_table(s)
    assert fast.allocator.free_block_count == public.allocator.free_block_count
    assert fast.allocator.allocate(3) == public.allocator.allocate(3)


def test_library_decode_plan_table():
    """nie_paged_decode_plan writes the host plan's work-item table: for 16
    sequences of 29,600 tokens the 16 splits of 116 tiles above, items in
    sequence order and each sequence's first item the splits before it; for
    ragged lengths ceil(tiles / split) items per sequence; for more sequences
    than a table holds a count and split length of 0 (the launch then plans
    from its bounds), which decode_plan_fits reports."""
    nbytes = _native.decode_plan_bytes()
    assert nbytes == 4 * (2 + 256 + 128 + 128)
    buf = np.zeros(nbytes // 4, dtype=np.int32)

    def plan(lens):
        lens = np.asarray(lens, dtype=np.int32)
        buf[:] = -1
        _native.write_decode_plan(buf.ctypes.data, nbytes, torch.bfloat16, 32, 8, 64, 16, lens, int(lens.max()),
                                  int(lens.sum()))
        count, tps = int(buf[0]), int(buf[1])
        items = [(int(i) >> 16, int(i) & 0xFFFF) for i in buf[2 : 2 + count].view(np.uint32)]
        return count, tps, items, buf[258 : 258 + len(lens)].tolist(), buf[386 : 386 + len(lens)].tolist()

    count, tps, items, seq_len, first = plan([29600] * 16)
    assert (count, tps) == (256, 116)
    assert items == [(b, s) for b in range(16) for s in range(16)]
    assert seq_len == [29600] * 16 and first == [16 * b for b in range(16)]

    lens = [17, 64, 129, 500, 3000]
    count, tps, items, seq_len, first = plan(lens)
    splits = [-(-(-(-n // 16)) // tps) for n in lens]
    assert tps >= 2 and count == sum(splits) and seq_len == lens
    assert first == [sum(splits[:b]) for b in range(len(lens))]
    assert items == [(b, s) for b in range(len(lens)) for s in range(splits[b])]
    assert _native.decode_plan_fits(torch.bfloat16, 32, 8, 64, 16, lens)

    count, tps, *_ = plan([100] * 130)
    assert (count, tps) == (0, 0)
    assert not _native.decode_plan_fits(torch.bfloat16, 32, 8, 64, 16, [100] * 130)
