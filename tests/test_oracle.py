"""Pins the oracle before it is trusted as the checker (CPU only).

Each oracle function is checked against something other than its own
formula: the reference tests' known answers, a brute-force float64 loop
written independently of the numpy closed form, special cases whose answer
the mathematics fixes, and invariants (block permutation, garbage past the
length, chunked == one-shot).  ``test_pins_catch_planted_mistakes`` plants
plausible mistakes in the oracle and shows that these pins fail on them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from nano_infer_engine import workloads
from nano_infer_engine.block_allocator import BlockAllocator
from nano_infer_engine.paged_cache import PagedKVCache
from oracle import closed_form, reference_ops, slots


# ---------------------------------------------------------------------------
# independent float64 brute force (pure Python loops, tiny inputs only)
# ---------------------------------------------------------------------------
def _brute_attention(q, k, v, q_positions, scale):
    tq, hq, d = len(q), len(q[0]), len(q[0][0])
    s, hkv = len(k), len(k[0])
    group = hq // hkv
    out = [[[0.0] * d for _ in range(hq)] for _ in range(tq)]
    for t in range(tq):
        for h in range(hq):
            kvh = h // group
            logits = []
            for j in range(s):
                if j <= q_positions[t]:
                    logits.append(sum(q[t][h][x] * k[j][kvh][x] for x in range(d)) * scale)
            top = max(logits)
            weights = [math.exp(x - top) for x in logits]
            total = sum(weights)
            for x in range(d):
                out[t][h][x] = sum(weights[j] * v[j][kvh][x] for j in range(len(weights))) / total
    return np.asarray(out)


def _tiny(seed, tq, s, hq, hkv, d):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((tq, hq, d)), rng.standard_normal((s, hkv, d)), rng.standard_normal((s, hkv, d)))


@pytest.mark.parametrize("hq,hkv", [(1, 1), (4, 2), (4, 1), (6, 3)])
def test_closed_form_matches_brute_force(hq, hkv):
    q, k, v = _tiny(hq * 10 + hkv, 3, 7, hq, hkv, 5)
    positions = [4, 5, 6]
    want = _brute_attention(q.tolist(), k.tolist(), v.tolist(), positions, 0.37)
    got = closed_form.attention(q, k, v, positions, 0.37)
    assert np.abs(got - want).max() < 1e-12


def test_closed_form_special_cases():
    q, k, v = _tiny(3, 1, 9, 4, 2, 6)
    # one visible key: the output is that key's value row exactly
    one = closed_form.attention(q, k, v, [0], 0.5)[0]
    for h in range(4):
        assert np.array_equal(one[h], v[0, h // 2])
    # identical keys: uniform weights, the output is the mean of V
    k_same = np.repeat(k[:1], 9, axis=0)
    mean = closed_form.attention(q, k_same, v, [8], 0.5)[0]
    for h in range(4):
        assert np.allclose(mean[h], v[:, h // 2].mean(axis=0), atol=1e-13)
    # scale 0 under a causal prefix: the mean of the visible values
    pref = closed_form.attention(q, k, v, [3], 0.0)[0]
    assert np.allclose(pref[1], v[:4, 0].mean(axis=0), atol=1e-13)
    # one dominant key takes all the weight
    k_dom = k.copy()
    k_dom[5] = 40.0 * q[0, 2][None]  # kv head 1 serves q heads 2, 3
    dom = closed_form.attention(q, k_dom, v, [8], 1.0)[0]
    assert np.allclose(dom[2], v[5, 1], atol=1e-9)


# ---------------------------------------------------------------------------
# decode oracle (paged_attention_reference restatement)
# ---------------------------------------------------------------------------
def _paged_layout(seed, lengths, block_size, hq, hkv, d, num_blocks, dtype=torch.float32, layers=2, layer=1):
    """Contiguous K/V per sequence scattered into a permuted pool; garbage elsewhere."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(num_blocks)
    pool_k = torch.from_numpy(rng.standard_normal((layers, num_blocks, block_size, hkv, d))).to(dtype)
    pool_v = torch.from_numpy(rng.standard_normal((layers, num_blocks, block_size, hkv, d))).to(dtype)
    tables, contig, cursor = [], [], 0
    for n in lengths:
        nb = slots.blocks_needed(n, block_size)
        table = [int(x) for x in perm[cursor : cursor + nb]]
        cursor += nb
        ks = torch.from_numpy(rng.standard_normal((n, hkv, d))).to(dtype)
        vs = torch.from_numpy(rng.standard_normal((n, hkv, d))).to(dtype)
        reference_ops.write_tokens(pool_k, pool_v, layer, table, block_size, 0, ks, vs)
        tables.append(tuple(table))
        contig.append((ks, vs))
    q = torch.from_numpy(rng.standard_normal((len(lengths), hq, d))).to(dtype)
    return pool_k, pool_v, tuple(tables), contig, q


def test_reference_decode_known_layout():
    """The reference test's layout: length 5, block_size 2, table (3, 0, 2), layer 1."""
    torch.manual_seed(0)
    q = torch.randn(4, 3)
    ks, vs = torch.randn(5, 2, 3), torch.randn(5, 2, 3)
    kc, vc = torch.randn(2, 4, 2, 2, 3), torch.randn(2, 4, 2, 2, 3)
    reference_ops.write_tokens(kc, vc, 1, (3, 0, 2), 2, 0, ks, vs)
    got = reference_ops.paged_attention_reference(q, kc, vc, (3, 0, 2), 5, 1)
    exact = closed_form.decode(q.numpy(), ks.numpy(), vs.numpy(), 3**-0.5)
    assert np.abs(got.numpy() - exact).max() < 1e-6


def test_reference_decode_matches_closed_form_fp32():
    lengths = [1, 2, 17, 64, 129]
    kc, vc, tables, contig, q = _paged_layout(11, lengths, 16, 8, 2, 64, 40)
    got = reference_ops.batched_paged_attention_reference(q, kc, vc, tables, tuple(lengths), 1)
    for b, (ks, vs) in enumerate(contig):
        exact = closed_form.decode(q[b].numpy(), ks.numpy(), vs.numpy(), 64**-0.5)
        assert np.abs(got[b].numpy() - exact).max() < 1e-5


def test_reference_decode_bf16_within_tolerance_of_float64():
    wl = workloads.decode_small()
    kc, vc = wl.pool(torch.bfloat16)
    q, _, _ = wl.new_tokens(torch.bfloat16)
    got = reference_ops.batched_paged_attention_reference(
        q, kc, vc, tuple(tuple(t) for t in wl.tables), tuple(wl.seq_lens), 0
    )
    worst = 0.0
    for b in range(4):
        ks, vs = reference_ops.gather_tokens(kc, vc, 0, wl.tables[b], wl.block_size, wl.seq_lens[b])
        exact = closed_form.decode(q[b].float().numpy(), ks.float().numpy(), vs.float().numpy(), 0.125)
        worst = max(worst, float(np.abs(got[b].float().numpy() - exact).max()))
    assert worst <= 2e-2


def test_reference_decode_invariants():
    lengths = [5, 33, 16]
    kc, vc, tables, contig, q = _paged_layout(5, lengths, 16, 4, 2, 64, 12)
    base = reference_ops.batched_paged_attention_reference(q, kc, vc, tables, tuple(lengths), 1)
    # length-1 sequence returns V exactly
    one = reference_ops.paged_attention_reference(q[0], kc, vc, tables[0], 1, 1)
    assert torch.equal(one, contig[0][1][0].repeat_interleave(2, dim=0))
    # relocating blocks (table rewritten to match) is bit-identical
    perm = torch.randperm(12, generator=torch.Generator().manual_seed(3))
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(12)
    kc2, vc2 = kc[:, perm], vc[:, perm]
    tables2 = tuple(tuple(int(inverse[b]) for b in t) for t in tables)
    moved = reference_ops.batched_paged_attention_reference(q, kc2, vc2, tables2, tuple(lengths), 1)
    assert torch.equal(base, moved)
    # garbage past each length (same block) has no effect
    kc3, vc3 = kc.clone(), vc.clone()
    for t, n in zip(tables, lengths):
        last = t[(n - 1) // 16]
        kc3[1, last, (n - 1) % 16 + 1 :] = float("nan")
        vc3[1, last, (n - 1) % 16 + 1 :] = float("nan")
    assert torch.equal(base, reference_ops.batched_paged_attention_reference(q, kc3, vc3, tables, tuple(lengths), 1))


# ---------------------------------------------------------------------------
# ragged (varlen chunked prefill) oracle
# ---------------------------------------------------------------------------
def _ragged_case(seed, ctx, qlen, hq=4, hkv=2, d=64, bs=16, dtype=torch.float32):
    wl = workloads.ragged(ctx, qlen, seed=seed, pool_factor=1.5, q_heads=hq, kv_heads=hkv, head_dim=d, block_size=bs)
    kc, vc = wl.pool(dtype)
    q, k, v = wl.new_tokens(dtype)
    return wl, kc, vc, q, k, v


def test_ragged_reference_matches_closed_form():
    wl, kc, vc, q, k, v = _ragged_case(21, [0, 3, 40, 0], [9, 5, 1, 17], bs=4)
    keys, values = kc.clone(), vc.clone()
    got = reference_ops.ragged_attention_reference(q, k, v, keys, values, 0, wl.tables, wl.context_lens,
                                                   wl.query_lens, 0.125)
    start = 0
    for table, c, n in zip(wl.tables, wl.context_lens, wl.query_lens):
        ks, vs = reference_ops.gather_tokens(keys, values, 0, table, 4, c + n)
        exact = closed_form.attention(q[start : start + n].numpy(), ks.numpy(), vs.numpy(), list(range(c, c + n)), 0.125)
        assert np.abs(got[start : start + n].numpy() - exact).max() < 1e-5
        # the chunk's own K/V went into the cache at slots ctx .. ctx+n-1
        assert torch.equal(ks[c:], k[start : start + n]) and torch.equal(vs[c:], v[start : start + n])
        start += n


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_timing_variants_of_the_oracle_agree_with_it(dtype):
    """The GPU-timing variants (batched matmuls over contiguous operands
    instead of einsum; indexed write / gather instead of per-token copies)
    compute the same values: the vectorized ragged oracle bit for bit on the
    CPU (same products on the same gathered tensors), the matmul decode loop
    within fp32 reassociation / one bf16 rounding of the einsum loop, and the
    closed form as a third witness."""
    lengths = [1, 17, 64, 129]
    kc, vc, tables, contig, q = _paged_layout(13, lengths, 16, 8, 2, 64, 40)
    kc, vc, q = kc.to(dtype), vc.to(dtype), q.to(dtype)
    a = reference_ops.batched_paged_attention_reference(q, kc, vc, tables, tuple(lengths), 1)
    b = reference_ops.batched_paged_attention_reference_matmul(q, kc, vc, tables, tuple(lengths), 1)
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert (a.float() - b.float()).abs().max().item() <= tol
    for i, (ks, vs) in enumerate(contig):
        exact = closed_form.decode(q[i].float().numpy(), ks.to(dtype).float().numpy(), vs.to(dtype).float().numpy(),
                                   64**-0.5)
        assert np.abs(b[i].float().numpy() - exact).max() < (1e-5 if dtype == torch.float32 else 2e-2)
    wl, kc, vc, q, k, v = _ragged_case(23, [0, 3, 40, 0], [9, 5, 1, 17], bs=4, dtype=dtype)
    k1, v1, k2, v2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    want = reference_ops.ragged_attention_reference(q, k, v, k1, v1, 0, wl.tables, wl.context_lens, wl.query_lens,
                                                    0.125)
    got = reference_ops.ragged_attention_reference_vectorized(q, k, v, k2, v2, 0, wl.tables, wl.context_lens,
                                                              wl.query_lens, 0.125)
    assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert torch.equal(got, want)


def test_ragged_chunked_equals_one_shot_and_decode_row_equals_decode():
    wl, kc, vc, q, k, v = _ragged_case(22, [0], [24], bs=4)
    one_k, one_v = kc.clone(), vc.clone()
    whole = reference_ops.ragged_attention_reference(q, k, v, one_k, one_v, 0, wl.tables, [0], [24], 0.125)
    two_k, two_v = kc.clone(), vc.clone()
    first = reference_ops.ragged_attention_reference(q[:10], k[:10], v[:10], two_k, two_v, 0, wl.tables, [0], [10], 0.125)
    rest = reference_ops.ragged_attention_reference(q[10:], k[10:], v[10:], two_k, two_v, 0, wl.tables, [10], [14], 0.125)
    assert torch.equal(one_k, two_k) and torch.equal(one_v, two_v)
    torch.testing.assert_close(torch.cat([first, rest]), whole, rtol=1e-6, atol=1e-6)
    # the last row (position 23) is a decode at length 24
    dec = reference_ops.paged_attention_reference(q[23], one_k, one_v, tuple(wl.tables[0]), 24, 0)
    torch.testing.assert_close(whole[23], dec, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# slot math, write / gather, allocator: the reference tests' known answers
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("tokens,blocks", [(1, 1), (4, 1), (5, 2), (8, 2), (9, 3)])
def test_blocks_needed_known_answers(tokens, blocks):
    assert slots.blocks_needed(tokens, 4) == blocks


def test_allocator_known_answers():
    assert slots.lifo_allocation_order(4, [("alloc", 2)]) == [[0, 1]]
    grants = slots.lifo_allocation_order(4, [("alloc", 4), ("free", 0)])
    assert grants[0] == [0, 1, 2, 3]
    # the reference frees [1, 3] of a full pool and gets [1, 3] back
    alloc = BlockAllocator(4)
    taken = alloc.allocate(4)
    alloc.free([taken[1], taken[3]])
    assert alloc.allocate(2) == [1, 3]
    # the oracle's LIFO model agrees with the allocator on a longer history
    history = [("alloc", 3), ("alloc", 2), ("free", 0), ("alloc", 4), ("free", 1), ("alloc", 1)]
    model = slots.lifo_allocation_order(9, history)
    real = BlockAllocator(9)
    granted: list[list[int]] = []
    for kind, arg in history:
        if kind == "alloc":
            granted.append(real.allocate(arg))
        else:
            real.free(granted[arg])
            granted.append([])
    assert granted == model


def test_fragmented_table_and_round_trip():
    """Reference known answer: three 1-block sequences, free the 1st and 3rd,
    then a 6-token sequence (block_size 4) gets table (2, 0)."""
    cache = PagedKVCache(6, 4, 2, 2, 4, torch.float32, "cpu")
    for sid in ("temporary-a", "temporary-b", "temporary-c"):
        cache.ensure_capacity(sid, 1)
    cache.release("temporary-a")
    cache.release("temporary-c")
    cache.ensure_capacity("request-a", 6)
    table = cache.get_block_table("request-a")
    assert table == (2, 0)
    keys = torch.arange(6 * 2 * 4, dtype=torch.float32).reshape(6, 2, 4)
    values = keys + 100
    pool_k = torch.zeros(2, 6, 4, 2, 4)
    pool_v = torch.zeros_like(pool_k)
    reference_ops.write_tokens(pool_k, pool_v, 1, table, 4, 0, keys, values)
    gk, gv = reference_ops.gather_tokens(pool_k, pool_v, 1, table, 4, 6)
    assert torch.equal(gk, keys) and torch.equal(gv, values)
    # positions 0-3 in block 2, 4-5 in block 0
    assert torch.equal(pool_k[1, 2], keys[:4]) and torch.equal(pool_k[1, 0, :2], keys[4:])
    flat = slots.slot_mapping([table], [0], [6], 4)
    assert flat.tolist() == [8, 9, 10, 11, 0, 1]
    assert cache.slots_for("request-a", 0, 6).tolist() == flat.tolist()


def test_slot_mapping_agrees_everywhere():
    wl = workloads.mixed_prefill()
    want = slots.slot_mapping(wl.tables, wl.context_lens, wl.query_lens, wl.block_size)
    assert np.array_equal(wl.slots(), want)
    with pytest.raises(IndexError, match="exceeds allocated capacity"):
        slots.resolve(wl.tables[0], len(wl.tables[0]) * wl.block_size, wl.block_size)


# ---------------------------------------------------------------------------
# algorithmic byte / flop figures used by the roofline
# ---------------------------------------------------------------------------
def test_workload_accounting_known_values():
    small = workloads.decode_small()
    assert small.seq_lens == [17, 64, 129, 500]
    assert sum(slots.blocks_needed(n, 16) for n in small.seq_lens) == 47
    assert workloads.decode_bytes(small.seq_lens) == 1_454_080 + 32_768 + 204
    assert workloads.decode_bytes([29600] * 16) == 970_182_336
    assert workloads.prefill_flops([0, 384, 1024, 4000], [128] * 4) == 4 * 32 * 64 * 725_248
    ctx = workloads.lognormal_lengths(1)
    assert len(ctx) == 16 and min(ctx) >= 32 and max(ctx) <= 29600
    assert sum(ctx) == 43_135


# ---------------------------------------------------------------------------
# planted mistakes: the pins above must reject each of these oracle mutants
# ---------------------------------------------------------------------------
def _mutant_decode(kind):
    def run(query, key_cache, value_cache, block_table, sequence_length, layer_index):
        _, _, bs, hkv, d = key_cache.shape
        group = query.shape[0] // hkv
        blocks = -(-sequence_length // bs)
        order = list(block_table[:blocks])
        if kind == "reversed_blocks":
            order = order[::-1]
        scores, values = [], []
        for logical, physical in enumerate(order):
            valid = min(bs, sequence_length - logical * bs)
            if kind == "whole_last_block":
                valid = bs
            if kind == "gqa_modulo":
                k_rows = key_cache[layer_index, physical, :valid].repeat(1, group, 1)
                v_rows = value_cache[layer_index, physical, :valid].repeat(1, group, 1)
            else:
                k_rows = key_cache[layer_index, physical, :valid].repeat_interleave(group, dim=1)
                v_rows = value_cache[layer_index, physical, :valid].repeat_interleave(group, dim=1)
            scale = 1.0 if kind == "no_scale" else d**-0.5
            scores.append(torch.einsum("hd,thd->ht", query, k_rows) * scale)
            values.append(v_rows)
        w = torch.softmax(torch.cat(scores, dim=-1), dim=-1, dtype=torch.float32).to(query.dtype)
        return torch.einsum("ht,thd->hd", w, torch.cat(values, dim=0))

    return run


@pytest.mark.parametrize("kind", ["gqa_modulo", "reversed_blocks", "whole_last_block", "no_scale"])
def test_pins_catch_planted_mistakes(kind, monkeypatch):
    monkeypatch.setattr(reference_ops, "paged_attention_reference", _mutant_decode(kind))
    lengths = [5, 33, 20]
    kc, vc, tables, contig, q = _paged_layout(5, lengths, 16, 4, 2, 64, 12)
    worst = 0.0
    for b, (ks, vs) in enumerate(contig):
        got = reference_ops.paged_attention_reference(q[b], kc, vc, tables[b], lengths[b], 1)
        exact = closed_form.decode(q[b].numpy(), ks.numpy(), vs.numpy(), 64**-0.5)
        worst = max(worst, float(np.nan_to_num(np.abs(got.numpy() - exact), nan=1e9).max()))
    assert worst > 1e-3, f"closed-form pin did not notice mutant {kind}"


# ---------------------------------------------------------------------------
# RoPE (layers/rope.py of the reference): frequencies, rotation, tables
# ---------------------------------------------------------------------------
_LLAMA3 = {"factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}


def _rope_float64(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor) -> np.ndarray:
    """Rotation of the pairs (i, i + D/2) by the fp32 angle p*f_i, in float64 (independent of torch's sin/cos)."""
    half = x.shape[-1] // 2
    angle = (positions.to(torch.float32)[:, None] * inv_freq).double().numpy()[:, None, :]
    xs = x.double().numpy()
    x1, x2 = xs[..., :half], xs[..., half:]
    return np.concatenate((x1 * np.cos(angle) - x2 * np.sin(angle), x2 * np.cos(angle) + x1 * np.sin(angle)), -1)


@pytest.mark.parametrize("dim", [64, 128])
def test_rope_inv_freq_closed_forms(dim):
    plain = reference_ops.rope_inv_freq(dim, 500000.0).double().numpy()
    exact = np.array([500000.0 ** (-2 * i / dim) for i in range(dim // 2)])
    assert plain[0] == 1.0 and np.allclose(plain, exact, rtol=2e-6, atol=0)
    scaled = reference_ops.rope_inv_freq(dim, 500000.0, _LLAMA3).double().numpy()
    bands = {"low": 0, "mid": 0, "high": 0}
    for f, got in zip(exact, scaled):
        wavelength = 2 * math.pi / f
        if wavelength > 8192:  # long wavelengths slowed by the factor
            want, band = f / 32.0, "low"
        elif wavelength < 2048:  # short ones kept
            want, band = f, "high"
        else:  # linear blend in 1/wavelength between the two
            smooth = (8192 / wavelength - 1.0) / 3.0
            want, band = (1 - smooth) * f / 32.0 + smooth * f, "mid"
        bands[band] += 1
        assert got == pytest.approx(want, rel=5e-6)
    assert all(bands.values()), bands  # every band is exercised


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_reference_matches_float64_rotation(dtype):
    g = torch.Generator().manual_seed(21)
    inv_freq = reference_ops.rope_inv_freq(64, 500000.0, _LLAMA3)
    positions = torch.tensor([0, 1, 7, 500, 4095, 8192, 29599, 131071], dtype=torch.int64)
    x = torch.randn((8, 3, 64), generator=g).to(dtype)
    got = reference_ops.rope_reference(x, positions, inv_freq)
    # position 0 is the identity, exactly
    assert torch.equal(got[0], x[0])
    tol = 1e-5 if dtype == torch.float32 else 6e-2
    assert np.abs(got.double().numpy() - _rope_float64(x, positions, inv_freq)).max() <= tol
    if dtype == torch.float32:  # rotations keep each pair's length
        half = 32
        n_in = x[..., :half] ** 2 + x[..., half:] ** 2
        n_out = got[..., :half] ** 2 + got[..., half:] ** 2
        assert torch.allclose(n_in, n_out, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("kind", ["sign", "interleaved", "no_scaling"])
def test_rope_pin_catches_planted_mistakes(kind):
    g = torch.Generator().manual_seed(22)
    inv_freq = reference_ops.rope_inv_freq(64, 500000.0, _LLAMA3)
    positions = torch.tensor([3, 100, 9000, 20000], dtype=torch.int64)
    x = torch.randn((4, 2, 64), generator=g)
    if kind == "no_scaling":
        got = reference_ops.rope_reference(x, positions, reference_ops.rope_inv_freq(64, 500000.0))
    else:
        angles = positions.float()[:, None] * inv_freq
        sin, cos = torch.sin(angles)[:, None], torch.cos(angles)[:, None]
        if kind == "sign":
            a, b = x[..., :32], x[..., 32:]
            got = torch.cat((a * cos + b * sin, b * cos - a * sin), -1)
        else:  # pairs (2i, 2i+1) instead of (i, i + D/2)
            a, b = x[..., 0::2], x[..., 1::2]
            got = torch.stack((a * cos - b * sin, b * cos + a * sin), -1).flatten(-2)
    assert np.abs(got.double().numpy() - _rope_float64(x, positions, inv_freq)).max() > 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("scaled", [False, True])
def test_product_rope_and_tables_match_oracle_bit_for_bit(dtype, scaled):
    from nano_infer_engine.layers.rope import Rope, RopeScale

    rope = RopeScale(64) if scaled else Rope(64)
    inv_freq = reference_ops.rope_module_inv_freq(rope, torch.device("cpu"))
    assert torch.equal(rope.inv_freq(torch.device("cpu")), inv_freq)
    g = torch.Generator().manual_seed(23)
    positions = torch.tensor([0, 5, 17, 4096, 9000, 12287], dtype=torch.int64)
    x = torch.randn((6, 4, 64), generator=g).to(dtype)
    assert torch.equal(rope.rotate_tokens(x, positions), reference_ops.rope_reference(x, positions, inv_freq))
    cos, sin = rope.tables(torch.device("cpu"), dtype, 12288)
    assert cos.shape == (12288, 32) and sin.shape == (12288, 32)
    angles = positions.float()[:, None] * inv_freq
    assert torch.equal(cos[positions], torch.cos(angles).to(dtype))
    assert torch.equal(sin[positions], torch.sin(angles).to(dtype))


def test_batched_product_is_the_matmul_on_the_cpu():
    """On the CPU the oracle's guarded product is ``a @ b`` for any layout."""
    gen = torch.Generator().manual_seed(0)
    a = torch.randn((3, 2, 8), generator=gen).to(torch.bfloat16)
    b = torch.randn((3, 5, 8), generator=gen).to(torch.bfloat16).transpose(-1, -2)
    assert torch.equal(reference_ops.batched_product(a, b), a @ b)
