"""Long-context decode (16 x 29600 tokens) and prefill over a pool beyond 2**31 elements.

The 16 x 29600 decode step with its per-step append (one fused
nie_paged_decode_append launch) runs on a 300,000-block pool: 2.46e9
elements per K / V tensor, so element offsets of the high blocks exceed
2**31.  Tables are a seeded permutation of the whole pool, and every other
sequence's newest block — the block the fused append writes — is forced
into the high range.  The output is checked against the oracle (the
reference's per-block loop, bf16, on the CPU over a compacted copy of the
used blocks) within the bf16 bar, and the appended rows bit for bit at their
slots.  The varlen prefill kernel is checked the same way on chunks whose
every block lies past 2**31 elements.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_infer_engine import _native
from oracle import reference_ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
NUM_BLOCKS, BS, HQ, HKV, D = 300_000, 16, 32, 8, 64
ROW = HKV * D
HIGH = 2**31 // (BS * ROW) + 1  # first block whose elements all sit past 2**31


def _log(msg: str) -> None:
    print(msg, flush=True)


@pytest.fixture(scope="module")
def pool():
    """(k, v) bf16 pools of NUM_BLOCKS blocks, zero; tests fill the blocks they use."""
    _log(f"large pool: {NUM_BLOCKS} blocks, {NUM_BLOCKS * BS * ROW / 1e9:.2f}e9 elements per tensor")
    k = torch.zeros((1, NUM_BLOCKS, BS, HKV, D), dtype=torch.bfloat16, device=DEV)
    v = torch.zeros_like(k)
    yield k, v
    del k, v
    torch.cuda.empty_cache()


def _fill(k, v, blocks: np.ndarray, seed: int) -> None:
    """N(0, 1) values into the given blocks of both pools."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    idx = torch.from_numpy(blocks.astype(np.int64)).to(DEV)
    shape = (1, len(blocks), BS, HKV, D)
    k[:, idx] = torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16)
    v[:, idx] = torch.randn(shape, generator=gen, device=DEV).to(torch.bfloat16)


def _compact(k, v, tables: list[list[int]]):
    """CPU copies of just the used blocks, and the tables renumbered into them."""
    used = np.unique(np.concatenate([np.asarray(t) for t in tables]))
    remap = {int(b): i for i, b in enumerate(used)}
    idx = torch.from_numpy(used.astype(np.int64)).to(DEV)
    return (k[:, idx].cpu(), v[:, idx].cpu(), tuple(tuple(remap[b] for b in t) for t in tables))


def _table_tensor(tables):
    width = max(len(t) for t in tables)
    arr = np.zeros((len(tables), width), dtype=np.int32)
    for r, t in enumerate(tables):
        arr[r, : len(t)] = t
    return torch.from_numpy(arr).to(DEV)


@pytest.mark.parametrize("host_plan", [True, False])
def test_decode_16x29600_with_append_on_pool_past_2_31(pool, host_plan):
    k, v = pool
    k.zero_()
    v.zero_()
    _log(f"decode 16x29600 + append, pool past 2**31, host_plan={host_plan}")
    rng = np.random.default_rng(4)
    ctx = 29600
    need = -(-(ctx + 1) // BS)  # blocks per sequence after the append
    perm = rng.permutation(NUM_BLOCKS)
    tables = [perm[i * need : (i + 1) * need].tolist() for i in range(16)]
    high = [int(b) for b in perm[16 * need :] if b >= HIGH]
    for i in range(0, 16, 2):  # the appended row of every other sequence lands past 2**31
        tables[i][-1] = high[i]
    assert sum(b >= HIGH for t in tables for b in t) > 1000
    used = np.asarray(sorted({b for t in tables for b in t}))
    _fill(k, v, used, seed=4)
    gen = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn((16, HQ, D), generator=gen, device=DEV).to(torch.bfloat16)
    k_new = torch.randn((16, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
    v_new = torch.randn((16, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
    lens = [ctx + 1] * 16
    # the oracle's copy is taken before the fused call writes the new rows
    k_small, v_small, small_tables = _compact(k, v, tables)
    out = _native.paged_decode(q, k, v, 0, _table_tensor(tables), torch.tensor(lens, dtype=torch.int32, device=DEV),
                               ctx + 1, 16 * (ctx + 1), D**-0.5, new_kv=(k_new, v_new),
                               seq_lens_host=lens if host_plan else None)
    torch.cuda.synchronize()
    flat_k, flat_v = k.view(-1, HKV, D), v.view(-1, HKV, D)
    for b, t in enumerate(tables):
        slot = t[ctx // BS] * BS + ctx % BS
        if b % 2 == 0:
            assert slot * ROW >= 2**31
        assert torch.equal(flat_k[slot], k_new[b]) and torch.equal(flat_v[slot], v_new[b]), b
    for b, t in enumerate(small_tables):
        reference_ops.write_tokens(k_small, v_small, 0, t, BS, ctx, k_new[b : b + 1].cpu(), v_new[b : b + 1].cpu())
    want = reference_ops.batched_paged_attention_reference(q.cpu(), k_small, v_small, small_tables, tuple(lens), 0)
    err = (out.cpu().float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= 2e-2


@pytest.mark.parametrize("host_plan", [True, False])
def test_varlen_prefill_on_blocks_past_2_31(pool, host_plan):
    k, v = pool
    _log(f"varlen prefill, every block past 2**31, host_plan={host_plan}")
    rng = np.random.default_rng(6)
    context_lens, query_lens = [4000, 0, 700], [128, 100, 1]
    need = [-(-(c + n) // BS) for c, n in zip(context_lens, query_lens)]
    chosen = HIGH + rng.permutation(NUM_BLOCKS - HIGH)[: sum(need)]
    tables, cursor = [], 0
    for n in need:
        tables.append([int(b) for b in chosen[cursor : cursor + n]])
        cursor += n
    _fill(k, v, np.asarray(chosen), seed=6)
    gen = torch.Generator(device=DEV).manual_seed(7)
    t = sum(query_lens)
    q = torch.randn((t, HQ, D), generator=gen, device=DEV).to(torch.bfloat16)
    k_new = torch.randn((t, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
    v_new = torch.randn((t, HKV, D), generator=gen, device=DEV).to(torch.bfloat16)
    k_small, v_small, small_tables = _compact(k, v, tables)
    slots = []
    for table, c, n in zip(tables, context_lens, query_lens):
        pos = np.arange(c, c + n)
        slots.append(np.asarray(table, dtype=np.int64)[pos // BS] * BS + pos % BS)
    slots = np.concatenate(slots)
    assert (slots * ROW >= 2**31).all()
    _native.kv_append(k, v, 0, k_new, v_new, torch.from_numpy(slots).to(DEV))
    cu = [0] + np.cumsum(query_lens).tolist()
    host = dict(cu_seqlens_host=cu, context_lens_host=context_lens) if host_plan else {}
    got = _native.varlen_prefill(q, torch.tensor(cu, dtype=torch.int64, device=DEV),
                                 torch.tensor(context_lens, dtype=torch.int32, device=DEV), k, v, 0,
                                 _table_tensor(tables), max(query_lens),
                                 max(c + n for c, n in zip(context_lens, query_lens)), D**-0.5, **host)
    torch.cuda.synchronize()
    want = reference_ops.ragged_attention_reference(q.cpu(), k_new.cpu(), v_new.cpu(), k_small, v_small, 0,
                                                    small_tables, context_lens, query_lens, D**-0.5)
    err = (got.cpu().float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= 2e-2
