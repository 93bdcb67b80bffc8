"""HIP kernels vs the oracle, called through the C ABI (via nano_infer_engine._native).

Bars: KV append / gather / block copies bit-exact; attention fp32 max-abs
<= 1e-4 and bf16 max-abs <= 2e-2 against the reference-algorithm oracle on
the same seeded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_infer_engine import _native, workloads
from oracle import reference_ops
from oracle import closed_form

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


def _log(msg: str) -> None:
    print(msg, flush=True)


@pytest.fixture(params=["reference", "fast"])
def rounding(request):
    """Both bf16 rounding points: the reference's (two passes, the default)
    and the one-pass online softmax (NIE_ROUND_FAST); fp32 calls are the
    same either way."""
    _native.set_attention_rounding(request.param)
    try:
        yield request.param
    finally:
        _native.set_attention_rounding("reference")


def _decode_hip(wl: workloads.PagedWorkload, kc, vc, q, dtype, host_plan=False):
    """The kernel's output.  host_plan: pass a host copy of the lengths (exact
    launch plan, work items in the kernel arguments)."""
    tables = torch.from_numpy(wl.table_array()).to(DEV)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)
    out = _native.paged_decode(
        q.to(DEV), kc, vc, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens), wl.head_dim**-0.5,
        seq_lens_host=list(wl.seq_lens) if host_plan else None,
    )
    torch.cuda.synchronize()
    return out.cpu()


def _decode_oracle(wl, kc_cpu, vc_cpu, q_cpu):
    return reference_ops.batched_paged_attention_reference(
        q_cpu, kc_cpu, vc_cpu, tuple(tuple(t) for t in wl.tables), tuple(wl.seq_lens), 0
    )


def test_oracle_refuses_bf16_batched_product_over_a_transposed_view():
    """The oracle's batched products on the GPU take contiguous right operands
    only in bf16 (the form that can fault is refused before any launch);
    contiguous operands and other dtypes go through unchanged."""
    a = torch.randn((4, 3, 8), device=DEV).to(torch.bfloat16)
    b = torch.randn((4, 5, 8), device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError, match="contiguous right operand"):
        reference_ops.batched_product(a, b.transpose(-1, -2))
    got = reference_ops.batched_product(a, b.transpose(-1, -2).contiguous())
    assert torch.equal(got, torch.matmul(a, b.transpose(-1, -2).contiguous()))
    f = reference_ops.batched_product(a.float(), b.float().transpose(-1, -2))
    assert f.shape == (4, 3, 5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kv_append_bit_exact(dtype):
    _log(f"kv_append dtype={dtype}")
    wl = workloads.ragged([0, 5, 31, 100], [7, 1, 16, 33], seed=11, num_blocks=64)
    kc, vc = wl.pool(dtype)
    _, k_new, v_new = wl.new_tokens(dtype)
    # source rows as a strided view of a wider buffer (like a fused projection output)
    wide_k = torch.zeros((k_new.shape[0], 3, wl.kv_heads, wl.head_dim), dtype=dtype)
    wide_k[:, 1] = k_new
    slots = wl.slots()
    slots_with_skip = np.concatenate([slots, [-1]])
    k_src = torch.cat([k_new, torch.full_like(k_new[:1], 7.0)])
    v_src = torch.cat([v_new, torch.full_like(v_new[:1], 7.0)])

    ref_k, ref_v = kc.clone(), vc.clone()
    start = 0
    for table, ctx, n in zip(wl.tables, wl.context_lens, wl.query_lens):
        reference_ops.write_tokens(ref_k, ref_v, 0, table, wl.block_size, ctx, k_new[start : start + n], v_new[start : start + n])
        start += n

    dk, dv = kc.to(DEV), vc.to(DEV)
    _native.kv_append(dk, dv, 0, k_src.to(DEV), v_src.to(DEV), torch.from_numpy(slots_with_skip).to(DEV))
    assert torch.equal(dk.cpu(), ref_k) and torch.equal(dv.cpu(), ref_v)

    # strided source view
    dk, dv = kc.to(DEV), vc.to(DEV)
    wide_k_dev = wide_k.to(DEV)
    _native.kv_append(dk, dv, 0, wide_k_dev[:, 1], v_new.to(DEV), torch.from_numpy(slots).to(DEV))
    assert torch.equal(dk.cpu(), ref_k) and torch.equal(dv.cpu(), ref_v)


def test_kv_append_large_pool_offsets():
    """Slots whose element offsets exceed 2**31 land exactly where the slot math says."""
    _log("kv_append large pool")
    num_blocks, bs, hkv, d = 270_000, 16, 8, 64  # 2.2e9 elements per pool (4.4 GB bf16)
    kc = torch.zeros((1, num_blocks, bs, hkv, d), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    # the last two slots sit past element offset 2**31; the final one is past
    # the pool and must be skipped
    slots = torch.tensor([0, 2**21 + 3, 2**31 // (hkv * d) + 5, num_blocks * bs - 1, num_blocks * bs], dtype=torch.int64)
    rows = (torch.arange(5 * hkv * d, dtype=torch.float32).reshape(5, hkv, d) + 1).to(torch.bfloat16)
    _native.kv_append(kc, vc, 0, rows.to(DEV), (rows + 1).to(DEV), slots.to(DEV))
    flat_k = kc.view(-1, hkv, d)
    flat_v = vc.view(-1, hkv, d)
    for i, s in enumerate(slots.tolist()[:4]):
        assert torch.equal(flat_k[s].cpu(), rows[i])
        assert torch.equal(flat_v[s].cpu(), rows[i] + 1)
    assert int((kc != 0).sum().item()) == 4 * hkv * d
    del kc, vc
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("block_size", [1, 4, 16, 32])
def test_kv_gather_bit_exact(dtype, block_size):
    _log(f"kv_gather dtype={dtype} bs={block_size}")
    wl = workloads.ragged([0], [45], seed=3, num_blocks=200 // block_size + 8, block_size=block_size)
    kc, vc = wl.pool(dtype)
    table = wl.tables[0]
    want_k, want_v = reference_ops.gather_tokens(kc, vc, 0, table, block_size, 45)
    got_k, got_v = _native.kv_gather(
        kc.to(DEV), vc.to(DEV), 0, torch.tensor(table, dtype=torch.int32, device=DEV), 45
    )
    assert torch.equal(got_k.cpu(), want_k) and torch.equal(got_v.cpu(), want_v)


def test_kv_copy_blocks_round_trip():
    _log("kv_copy_blocks")
    shape = (3, 20, 16, 8, 64)
    g = torch.Generator().manual_seed(5)
    src_k = torch.randn(shape, generator=g).to(torch.bfloat16)
    src_v = torch.randn(shape, generator=g).to(torch.bfloat16)
    blocks = [7, 2, 19, 0]
    staged_k = torch.empty((3, 4, 16, 8, 64), dtype=torch.bfloat16, device=DEV)
    staged_v = torch.empty_like(staged_k)
    _native.kv_copy_blocks(src_k.to(DEV), src_v.to(DEV), torch.tensor(blocks, dtype=torch.int32, device=DEV),
                           staged_k, staged_v, None, 4)
    assert torch.equal(staged_k.cpu(), src_k[:, blocks]) and torch.equal(staged_v.cpu(), src_v[:, blocks])
    dst_k = torch.zeros((3, 10, 16, 8, 64), dtype=torch.bfloat16, device=DEV)
    dst_v = torch.zeros_like(dst_k)
    dst_blocks = [9, 1, 4, 3]
    _native.kv_copy_blocks(staged_k, staged_v, None, dst_k, dst_v, torch.tensor(dst_blocks, dtype=torch.int32, device=DEV), 4)
    assert torch.equal(dst_k[:, dst_blocks].cpu(), src_k[:, blocks])
    assert torch.equal(dst_v[:, dst_blocks].cpu(), src_v[:, blocks])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("q_heads,kv_heads,head_dim", [(32, 8, 64), (8, 2, 128)])
def test_rope_kv_append_bit_exact(dtype, q_heads, kv_heads, head_dim):
    """Fused RoPE + append == the oracle's RoPE (torch ops, same device) + slot writes, bit for bit.

    q/k/v are strided views of one (tokens, Hq + 2*Hkv, D) buffer, as a
    fused QKV projection produces; one token has slot -1 (skipped) and the
    positions reach the end of a 29600-token context.
    """
    from nano_infer_engine.layers.rope import RopeScale

    _log(f"rope_kv_append {dtype} hq={q_heads} hkv={kv_heads} d={head_dim}")
    gen = torch.Generator(device=DEV).manual_seed(31)
    tokens, num_blocks, bs, layers, layer = 37, 64, 16, 2, 1
    qkv = torch.randn((tokens, q_heads + 2 * kv_heads, head_dim), generator=gen, device=DEV).to(dtype)
    q, k, v = qkv[:, :q_heads], qkv[:, q_heads : q_heads + kv_heads], qkv[:, q_heads + kv_heads :]
    positions = torch.randint(0, 29600, (tokens,), generator=gen, device=DEV, dtype=torch.int64)
    positions[:3] = torch.tensor([0, 1, 29599], device=DEV)
    slots = torch.randperm(num_blocks * bs, generator=gen, device=DEV)[:tokens].to(torch.int64)
    slots[5] = -1
    kc = torch.randn((layers, num_blocks, bs, kv_heads, head_dim), generator=gen, device=DEV).to(dtype)
    vc = torch.randn_like(kc)

    rope = RopeScale(head_dim)
    inv_freq = reference_ops.rope_module_inv_freq(rope, DEV)
    q_want = reference_ops.rope_reference(q, positions, inv_freq)
    k_want = reference_ops.rope_reference(k, positions, inv_freq)
    kc_want, vc_want = kc.clone(), vc.clone()
    keep = slots >= 0
    kc_want[layer].view(-1, kv_heads, head_dim)[slots[keep]] = k_want[keep]
    vc_want[layer].view(-1, kv_heads, head_dim)[slots[keep]] = v[keep]

    cos, sin = rope.tables(DEV, dtype, 29600)
    k_before, v_before = k.clone(), v.clone()
    _native.rope_kv_append(kc, vc, layer, q, k, v, positions, slots, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q, q_want)
    assert torch.equal(kc, kc_want) and torch.equal(vc, vc_want)
    # k and v inputs are left as they were
    assert torch.equal(k, k_before) and torch.equal(v, v_before)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_small_matches_oracle(dtype, rounding):
    _log(f"decode_small dtype={dtype}")
    wl = workloads.decode_small()
    kc, vc = wl.pool(dtype)
    q, _, _ = wl.new_tokens(dtype)
    got = _decode_hip(wl, kc.to(DEV), vc.to(DEV), q, dtype)
    want = _decode_oracle(wl, kc, vc, q)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]
    if dtype == torch.float32:
        # and the oracle itself against float64 closed form
        for b in range(4):
            ks, vs = reference_ops.gather_tokens(kc, vc, 0, wl.tables[b], wl.block_size, wl.seq_lens[b])
            exact = closed_form.decode(q[b].numpy(), ks.numpy(), vs.numpy(), wl.head_dim**-0.5)
            assert np.abs(got[b].numpy() - exact).max() <= 1e-4


@pytest.mark.parametrize("host_plan", [False, True])
def test_decode_ragged_lognormal_bf16(host_plan, rounding):
    """16 sequences, lognormal lengths up to 29600 (split-K with merge);
    launches planned from bounds and from host lengths."""
    _log(f"decode_ragged bf16 host_plan={host_plan}")
    wl = workloads.decode_ragged()
    kc, vc = wl.pool(torch.bfloat16)
    q, _, _ = wl.new_tokens(torch.bfloat16)
    got = _decode_hip(wl, kc.to(DEV), vc.to(DEV), q, torch.bfloat16, host_plan)
    want = _decode_oracle(wl, kc, vc, q)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  lengths={wl.seq_lens} max_abs_err={err:.3e}")
    assert err <= 2e-2


@pytest.mark.parametrize(
    "q_heads,kv_heads,head_dim,block_size",
    [(4, 4, 64, 16), (4, 2, 64, 2), (8, 2, 64, 1), (16, 2, 64, 4), (16, 1, 64, 32), (32, 8, 128, 16), (8, 8, 128, 3)],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("host_plan", [False, True])
def test_decode_shapes(q_heads, kv_heads, head_dim, block_size, dtype, host_plan, rounding):
    _log(f"decode shapes hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype} host_plan={host_plan}")
    wl = workloads.ragged([0, 4, 70, 300, 1000], [1] * 5, seed=7, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    kc, vc = wl.pool(dtype)
    q, _, _ = wl.new_tokens(dtype)
    got = _decode_hip(wl, kc.to(DEV), vc.to(DEV), q, dtype, host_plan)
    want = _decode_oracle(wl, kc, vc, q)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


def test_decode_ignores_garbage_past_length():
    """NaN in unused slots of the last block must not reach the output."""
    _log("decode garbage")
    wl = workloads.ragged([20, 37], [1, 1], seed=9, num_blocks=16)
    kc, vc = wl.pool(torch.bfloat16)
    for table, n in zip(wl.tables, wl.seq_lens):
        last = table[(n - 1) // 16]
        kc[0, last, (n - 1) % 16 + 1 :] = float("nan")
        vc[0, last, (n - 1) % 16 + 1 :] = float("nan")
    q, _, _ = wl.new_tokens(torch.bfloat16)
    got = _decode_hip(wl, kc.to(DEV), vc.to(DEV), q, torch.bfloat16)
    assert torch.isfinite(got).all()
    want = _decode_oracle(wl, kc, vc, q)
    assert (got.float() - want.float()).abs().max().item() <= 2e-2


def _control_regions_zero() -> bool:
    """Every cached workspace's control region (the one-launch decode's counters) is zero."""
    ctl = _native.workspace_control_bytes()
    # the region's last 128-byte line only counts waits that gave up
    return all(int(ws[: ctl - 128].count_nonzero().item()) == 0 for ws in _native._decode_workspaces.values())


def test_decode_tolerates_stale_workspace():
    """Past its control region the decode workspace needs no clearing: a
    workspace full of garbage there (random bytes, all ones, small
    integers), or one just overwritten by a prefill call's partials, gives
    correct output, and every call leaves the control region zero."""
    _log("decode stale workspace")
    wl = workloads.decode_ragged(seed=5)
    kc, vc = wl.pool(torch.bfloat16)
    q, _, _ = wl.new_tokens(torch.bfloat16)
    want = _decode_oracle(wl, kc, vc, q)
    dk, dv, dq = kc.to(DEV), vc.to(DEV), q.to(DEV)
    tables = torch.from_numpy(wl.table_array()).to(DEV)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)

    def run():
        out = _native.paged_decode(dq, dk, dv, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens),
                                   wl.head_dim**-0.5)
        torch.cuda.synchronize()
        return (out.cpu().float() - want.float()).abs().max().item()

    run()  # creates the cached workspace
    assert _control_regions_zero()
    ctl = _native.workspace_control_bytes()
    gen = torch.Generator(device=DEV).manual_seed(0)
    fills = {
        "random": lambda w: w.copy_(torch.randint(0, 256, w.shape, generator=gen, device=DEV, dtype=torch.uint8)),
        "ones": lambda w: w.fill_(255),
        "small integers": lambda w: w[: w.numel() // 8 * 8].view(torch.int64).copy_(
            torch.arange(w.numel() // 8, device=DEV, dtype=torch.int64) % 7 + 1),
    }
    for name, fill in fills.items():
        with torch.inference_mode():  # cached workspaces may have been made under inference mode
            for ws in _native._decode_workspaces.values():
                fill(ws[ctl:])
        err = run()
        _log(f"  {name}: max_abs_err={err:.3e}")
        assert err <= 2e-2
        assert _control_regions_zero()
    # a split-key prefill writes its partials over the same workspace
    pwl = workloads.ragged([3000, 40], [64, 1], seed=11)
    _prefill_case(pwl, torch.bfloat16)
    assert _control_regions_zero()
    err = run()
    _log(f"  after prefill: max_abs_err={err:.3e}")
    assert err <= 2e-2
    assert _control_regions_zero()


def test_decode_workspace_reuse_across_calls():
    """Back-to-back launches share one workspace: what a call leaves behind
    must not disturb the next call.

    Calls alternate between a long-context batch (many splits per sequence)
    and a short one, with no host synchronisation between them; every output
    is checked against the oracle afterwards.
    """
    _log("decode workspace reuse")
    cases = [workloads.decode_ragged(seed=s) for s in (1, 3)] + [workloads.decode_small()]
    prepared = []
    for wl in cases:
        kc, vc = wl.pool(torch.bfloat16)
        q, _, _ = wl.new_tokens(torch.bfloat16)
        prepared.append((wl, kc, vc, q, kc.to(DEV), vc.to(DEV), q.to(DEV),
                         torch.from_numpy(wl.table_array()).to(DEV),
                         torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)))
    outs = []
    for rep in range(3):
        for wl, _, _, _, dk, dv, dq, tables, lens in prepared:
            outs.append(_native.paged_decode(dq, dk, dv, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens),
                                             wl.head_dim**-0.5))
    torch.cuda.synchronize()
    for i, got in enumerate(outs):
        wl, kc, vc, q = prepared[i % len(prepared)][:4]
        err = (got.cpu().float() - _decode_oracle(wl, kc, vc, q).float()).abs().max().item()
        _log(f"  call {i} max_abs_err={err:.3e}")
        assert err <= 2e-2


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Bitwise equality (NaN slots compare equal to themselves)."""
    ints = {torch.bfloat16: torch.int16, torch.float32: torch.int32}[a.dtype]
    return a.dtype == b.dtype and torch.equal(a.cpu().view(ints), b.cpu().view(ints))


def _append_decode_pair(wl, dtype, host_plan, layer=0, table_edit=None, rope=False, pool_edit=None):
    """Fused append + decode against nie_kv_append then nie_paged_decode on the
    same inputs: caches and outputs must be bit-identical, and the output
    within tolerance of the oracle (which writes the rows, then attends).

    The pool gets `layer` extra leading layers of other values, so the
    fused write is checked at a layer offset; table_edit(table_array) may
    alter the device tables (both paths see the same ones).  rope: the fused
    call also rotates q and the new keys, against nie_rope_kv_append then
    nie_paged_decode.  pool_edit(kc, vc) may alter the pool first.
    """
    kc, vc = wl.pool(dtype)
    if pool_edit is not None:
        pool_edit(kc, vc)
    if layer:
        kc = torch.cat([torch.randn((layer,) + kc.shape[1:]).to(dtype), kc])
        vc = torch.cat([torch.randn((layer,) + vc.shape[1:]).to(dtype), vc])
    q, k_new, v_new = wl.new_tokens(dtype)
    table_arr = wl.table_array()
    if table_edit is not None:
        table_edit(table_arr)
    pos = np.asarray(wl.seq_lens) - 1
    slots = table_arr[np.arange(len(pos)), pos // wl.block_size].astype(np.int64) * wl.block_size + pos % wl.block_size
    tables = torch.from_numpy(table_arr).to(DEV)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)
    host = list(wl.seq_lens) if host_plan else None
    args = (max(wl.seq_lens), sum(wl.seq_lens), wl.head_dim**-0.5)
    dq, dkn, dvn = q.to(DEV), k_new.to(DEV), v_new.to(DEV)

    k1, v1 = kc.to(DEV), vc.to(DEV)
    tables_rope = None
    if rope:
        from nano_infer_engine.layers.rope import RopeScale

        tables_rope = RopeScale(wl.head_dim).tables(DEV, dtype, max(wl.seq_lens))
        q1 = dq.clone()
        positions = torch.from_numpy(pos.astype(np.int64)).to(DEV)
        _native.rope_kv_append(k1, v1, layer, q1, dkn, dvn, positions, torch.from_numpy(slots).to(DEV),
                               *tables_rope)
    else:
        q1 = dq
        _native.kv_append(k1, v1, layer, dkn, dvn, torch.from_numpy(slots).to(DEV))
    out1 = _native.paged_decode(q1, k1, v1, layer, tables, lens, *args, seq_lens_host=host)
    k2, v2 = kc.to(DEV), vc.to(DEV)
    q2 = dq.clone()
    out2 = _native.paged_decode(q2, k2, v2, layer, tables, lens, *args, seq_lens_host=host, new_kv=(dkn, dvn),
                                rope_tables=tables_rope)
    torch.cuda.synchronize()
    assert torch.equal(q2, dq), "the fused call must not modify q"
    assert _same_bits(k1, k2) and _same_bits(v1, v2), "fused write differs"
    assert _same_bits(out1, out2), "fused output differs"
    return out2.cpu(), kc, vc, q, k_new, v_new


@pytest.mark.parametrize(
    "q_heads,kv_heads,head_dim,block_size",
    [(32, 8, 64, 16), (4, 2, 64, 16), (4, 2, 64, 2), (16, 2, 64, 4), (16, 1, 64, 32), (32, 8, 128, 16),
     (8, 8, 128, 3)],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("host_plan", [False, True])
def test_decode_append_matches_append_then_decode(q_heads, kv_heads, head_dim, block_size, dtype, host_plan, rounding):
    """The new token lands on every row of a 16-key tile (contexts 0, 4, 15,
    16, 70, 300, 1000) and in single- and multi-split sequences."""
    _log(f"decode_append hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype} host_plan={host_plan}")
    wl = workloads.ragged([0, 4, 15, 16, 70, 300, 1000], [1] * 7, seed=13, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    got, kc, vc, q, k_new, v_new = _append_decode_pair(wl, dtype, host_plan, layer=1)
    ref_k, ref_v = kc.clone(), vc.clone()
    for b, (table, ctx) in enumerate(zip(wl.tables, wl.context_lens)):
        reference_ops.write_tokens(ref_k, ref_v, 1, table, wl.block_size, ctx, k_new[b : b + 1], v_new[b : b + 1])
    want = reference_ops.batched_paged_attention_reference(
        q, ref_k, ref_v, tuple(tuple(t) for t in wl.tables), tuple(wl.seq_lens), 1)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("host_plan", [False, True])
def test_decode_append_ragged_lognormal_bf16(host_plan):
    """The 16-sequence lognormal decode step (many splits per sequence)."""
    _log(f"decode_append ragged host_plan={host_plan}")
    wl = workloads.decode_ragged()
    _append_decode_pair(wl, torch.bfloat16, host_plan)


@pytest.mark.parametrize(
    "q_heads,kv_heads,head_dim,block_size",
    [(32, 8, 64, 16), (4, 2, 64, 16), (16, 2, 64, 4), (32, 8, 128, 16), (8, 8, 128, 3)],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("host_plan", [False, True])
def test_decode_rope_append_matches_rope_append_then_decode(q_heads, kv_heads, head_dim, block_size, dtype,
                                                           host_plan, rounding):
    """Fused RoPE + append + decode == nie_rope_kv_append then nie_paged_decode,
    caches and outputs bit for bit, q left unrotated."""
    _log(f"decode_rope_append hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype} "
         f"host_plan={host_plan}")
    wl = workloads.ragged([0, 4, 15, 16, 70, 300, 1000], [1] * 7, seed=19, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    _append_decode_pair(wl, dtype, host_plan, layer=1, rope=True)


@pytest.mark.parametrize("rope", [False, True])
def test_decode_append_ignores_stale_slot_content(rope, rounding):
    """NaN in the new token's slot and in every later slot of its block (what
    an unwritten pool may hold): the fused call's reads of those slots are
    replaced by the new row, so the output is finite and bit-identical to the
    separate calls, which write the slot first."""
    _log(f"decode_append stale slots rope={rope}")
    wl = workloads.ragged([40, 100, 7, 3000], [1, 1, 1, 1], seed=23, q_heads=32, kv_heads=8)

    def poison(kc, vc):
        for table, n in zip(wl.tables, wl.seq_lens):
            block = table[(n - 1) // wl.block_size]
            kc[0, block, (n - 1) % wl.block_size :] = float("nan")
            vc[0, block, (n - 1) % wl.block_size :] = float("nan")

    got = _append_decode_pair(wl, torch.bfloat16, False, rope=rope, pool_edit=poison)[0]
    assert torch.isfinite(got.float()).all()


def test_decode_append_skips_out_of_pool_table_entry():
    """A newest-token table entry outside the pool: no write (as kv_append
    skips an out-of-range slot), and the same output as the separate calls."""
    _log("decode_append out-of-pool entry")
    wl = workloads.ragged([40, 100, 7], [1, 1, 1], seed=17, q_heads=32, kv_heads=8)

    def edit(arr):
        arr[1, 100 // wl.block_size] = wl.num_blocks + 3

    _append_decode_pair(wl, torch.bfloat16, True, table_edit=edit)


def _prefill_case(wl, dtype, host_plan=True):
    """The kernel's output and the oracle's.  host_plan: pass host copies of
    the lengths (exact launch plan) or not (plan from upper bounds)."""
    kc, vc = wl.pool(dtype)
    q, k_new, v_new = wl.new_tokens(dtype)
    ref_k, ref_v = kc.clone(), vc.clone()
    want = reference_ops.ragged_attention_reference(
        q, k_new, v_new, ref_k, ref_v, 0, wl.tables, wl.context_lens, wl.query_lens, wl.head_dim**-0.5
    )
    dk, dv = kc.to(DEV), vc.to(DEV)
    _native.kv_append(dk, dv, 0, k_new.to(DEV), v_new.to(DEV), torch.from_numpy(wl.slots()).to(DEV))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(wl.query_lens)]), dtype=torch.int64, device=DEV)
    ctx = torch.tensor(wl.context_lens, dtype=torch.int32, device=DEV)
    tables = torch.from_numpy(wl.table_array()).to(DEV)
    host = dict(cu_seqlens_host=cu.cpu().tolist(), context_lens_host=list(wl.context_lens)) if host_plan else {}
    got = _native.varlen_prefill(q.to(DEV), cu, ctx, dk, dv, 0, tables, max(wl.query_lens), max(wl.seq_lens),
                                 wl.head_dim**-0.5, **host)
    torch.cuda.synchronize()
    assert torch.equal(dk.cpu(), ref_k) and torch.equal(dv.cpu(), ref_v)
    return got.cpu(), want


@pytest.mark.parametrize("host_plan", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_varlen_prefill_mixed_batch(dtype, host_plan, rounding):
    _log(f"varlen mixed {dtype} host_plan={host_plan}")
    wl = workloads.mixed_prefill()
    got, want = _prefill_case(wl, dtype, host_plan)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("which", ["prefill_prompts", "prefill_long_context"])
def test_varlen_prefill_long_workloads(which, rounding):
    """The long-prefill workloads the bench times: 4 fresh 2048-token prompts
    (64 query tiles per request, causal) and 4 chunks of 512 tokens on
    8192-token contexts, bf16, launches planned from host lengths."""
    _log(f"varlen long {which}")
    wl = getattr(workloads, which)()
    got, want = _prefill_case(wl, torch.bfloat16, True)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("host_plan", [True, False])
@pytest.mark.parametrize("block_size", [16, 64, 8])
def test_varlen_prefill_pieces_past_one_table_window(block_size, host_plan, dtype, rounding):
    """Pieces of more than 128 key tiles, whose blocks pass the first
    128-entry block-table window a wave holds (the kernel then queues up to
    five windows and moves them up as its lookups pass each one; with 8-key
    blocks every lane reads its own entries): chunks on 3000 to 9000-token
    contexts, planned from host lengths (a few long pieces per query tile)
    and from bounds (uniform pieces of about 150 tiles)."""
    if dtype == torch.float32 and rounding != "reference":
        pytest.skip("fp32 has one rounding")
    _log(f"varlen long pieces bs={block_size} host_plan={host_plan} {dtype}")
    wl = workloads.ragged([8192, 6000, 3000, 9000], [512, 256, 64, 128], seed=33, pool_factor=1.2,
                          block_size=block_size)
    got, want = _prefill_case(wl, dtype, host_plan)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("host_plan", [True, False])
def test_varlen_prefill_long_context_planned_from_bounds(host_plan, rounding):
    """The 4 x 512 chunks on 8192-token contexts with and without host
    lengths: one 544-tile piece per query tile, or uniform pieces of about
    150 tiles located on the device."""
    _log(f"varlen long context host_plan={host_plan}")
    got, want = _prefill_case(workloads.prefill_long_context(), torch.bfloat16, host_plan)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[torch.bfloat16]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_varlen_prefill_requests_past_index_255(dtype):
    """260 empty requests before four real ones: the real requests' query
    tiles carry request indices above 255, which the kernel-argument item
    table cannot encode, so the host plan must fall back to uniform pieces
    (whose merge jobs match what the kernel locates) rather than a balanced
    plan; the output matches the oracle."""
    _log(f"varlen prefill, requests past index 255, {dtype}")
    ctx = [16] * 260 + [3000, 0, 1200, 5000]
    qlen = [0] * 260 + [128, 128, 64, 1]
    wl = workloads.ragged(ctx, qlen, seed=31, pool_factor=1.2)
    got, want = _prefill_case(wl, dtype)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("context,query", [(300, 16), (600, 8), (1000, 40), (20000, 16)])
@pytest.mark.parametrize("host_plan", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_varlen_prefill_merge_batches(dtype, host_plan, context, query):
    """One request over one KV head, its keys split into about 3, 5, 9 and
    157 pieces (8 key tiles each): the merge loads its splits in batches of
    4, 8 or 16 chosen from the call's largest split count, and 157 splits
    take ten batches of 16 combined through the running maximum."""
    _log(f"varlen merge batches ctx={context} q={query} {dtype} host_plan={host_plan}")
    wl = workloads.ragged([context], [query], seed=31, pool_factor=1.2, q_heads=4, kv_heads=1, head_dim=64,
                          block_size=16)
    got, want = _prefill_case(wl, dtype, host_plan)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize(
    "q_heads,kv_heads,head_dim,block_size",
    [(4, 4, 64, 16), (4, 2, 64, 2), (8, 1, 64, 4), (16, 1, 64, 16), (32, 2, 128, 32), (8, 4, 128, 5)],
)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_varlen_prefill_shapes(q_heads, kv_heads, head_dim, block_size, dtype, rounding):
    _log(f"varlen shapes hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype}")
    wl = workloads.ragged([0, 3, 50, 0, 17], [19, 5, 1, 40, 2], seed=13, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    got, want = _prefill_case(wl, dtype)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize(
    "q_heads,kv_heads,head_dim,block_size",
    [(4, 4, 64, 16), (8, 4, 64, 16), (16, 4, 64, 8), (32, 4, 64, 16), (32, 8, 128, 16), (16, 1, 128, 32)],
)
@pytest.mark.parametrize("host_plan", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_varlen_prefill_split_keys(q_heads, kv_heads, head_dim, block_size, dtype, host_plan, rounding):
    """Contexts long enough that query tiles are split over several workgroups
    (at least 8 key tiles per split) and merged, next to short requests and
    decode rows; launches planned from host lengths and from bounds."""
    _log(f"varlen split hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype} host_plan={host_plan}")
    wl = workloads.ragged([700, 0, 300, 1500, 33], [70, 130, 1, 9, 64], seed=17, pool_factor=1.3, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    got, want = _prefill_case(wl, dtype, host_plan)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


def _rms_norm_reference(x, weight, eps):
    """The reference's RmsNorm.forward arithmetic (layers/rms_norm.py:25-31), fp32 on the CPU."""
    h = x.float()
    h = h / torch.sqrt(torch.mean(torch.square(h), dim=-1, keepdim=True) + eps)
    if weight is not None:
        h = weight.float() * h
    return h.to(x.dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rows,cols", [(1, 2048), (16, 2048), (37, 4096), (5, 64), (3, 8)])
@pytest.mark.parametrize("with_weight", [True, False])
@pytest.mark.parametrize("with_residual", [False, True])
def test_rms_norm_matches_reference_formula(dtype, rows, cols, with_weight, with_residual):
    """nie_rms_norm against the reference formula in fp32 on the CPU: the
    residual sum bit for bit; the normalised rows to one storage-dtype
    rounding (the sum of squares is reduced in another order)."""
    _log(f"rms_norm {dtype} rows={rows} cols={cols} weight={with_weight} residual={with_residual}")
    gen = torch.Generator().manual_seed(rows * 1000 + cols)
    x = (torch.randn((rows, cols), generator=gen) * 3).to(dtype)
    res = (torch.randn((rows, cols), generator=gen)).to(dtype) if with_residual else None
    w = (1 + 0.1 * torch.randn(cols, generator=gen)).to(dtype) if with_weight else None
    if res is not None:
        s_got, got = _native.rms_norm(x.to(DEV), None if w is None else w.to(DEV), 1e-5, residual=res.to(DEV))
        s_want = x + res
        assert torch.equal(s_got.cpu(), s_want)
        want = _rms_norm_reference(s_want, w, 1e-5)
    else:
        got = _native.rms_norm(x.to(DEV), None if w is None else w.to(DEV), 1e-5)
        want = _rms_norm_reference(x, w, 1e-5)
    torch.cuda.synchronize()
    got = got.cpu().float()
    want = want.float()
    rel = 2.0**-7 if dtype == torch.bfloat16 else 1e-5
    err = ((got - want).abs() / want.abs().clamp_min(1e-3)).max().item()
    mism = (got != want).float().mean().item()
    _log(f"  max_rel_err={err:.3e} mismatching={mism:.4f}")
    assert err <= rel
    if dtype == torch.bfloat16:
        assert mism < 0.01


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("halves", [False, True])
def test_silu_mul_matches_reference_formula(dtype, halves):
    """nie_silu_mul against F.silu(gate) * up computed in fp32 on the CPU with
    torch's roundings (silu rounded to the storage dtype, then the product);
    halves: gate and up are the two column halves of one (16, 16384) tensor,
    as a fused gate/up projection produces them."""
    _log(f"silu_mul {dtype} halves={halves}")
    gen = torch.Generator().manual_seed(5)
    g = (torch.randn((16, 8192), generator=gen) * 4).to(dtype)
    u = torch.randn((16, 8192), generator=gen).to(dtype)
    if halves:
        gu = torch.cat((g, u), dim=1).to(DEV)
        dg, du = gu.split((8192, 8192), dim=1)
    else:
        dg, du = g.to(DEV), u.to(DEV)
    got = _native.silu_mul(dg, du)
    torch.cuda.synchronize()
    want = (torch.nn.functional.silu(g.float()).to(dtype).float() * u.float()).to(dtype)
    got = got.cpu().float()
    want = want.float()
    rel = 2.0**-7 if dtype == torch.bfloat16 else 1e-6
    err = ((got - want).abs() / want.abs().clamp_min(1e-3)).max().item()
    mism = (got != want).float().mean().item()
    _log(f"  max_rel_err={err:.3e} mismatching={mism:.5f}")
    assert err <= rel
    if dtype == torch.bfloat16:
        assert mism < 0.001


def _linear_inputs(rows, n, k, seed, x_cols=None):
    gen = torch.Generator().manual_seed(seed)
    x_full = torch.randn((rows, x_cols or k), generator=gen).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=gen) / k**0.5).to(torch.bfloat16)
    return x_full, w


@pytest.mark.parametrize("rows", [1, 5, 16])
@pytest.mark.parametrize("n,k", [(3072, 2048), (2048, 8192), (1024, 4096), (32768, 2048)])
def test_linear_rows_matches_float64_product(rows, n, k):
    """nie_linear_rows against x . W^T in float64 on the CPU, rounded to bf16:
    every output within half a bf16 ulp of the exact product (plus the fp32
    accumulation's error), at most 1% of outputs one ulp away from torch's own
    bf16 GEMM on the GPU.  k = 2048, 4096 and 8192 are the kernel's 2-, 4- and
    8-pass builds; x is a column slice of a wider tensor (row stride > k)."""
    _log(f"linear_rows rows={rows} n={n} k={k}")
    x_full, w = _linear_inputs(rows, n, k, seed=rows * 7 + n, x_cols=k + 64)
    x = x_full[:, 32:32 + k]
    dx, dw = x_full.to(DEV)[:, 32:32 + k], w.to(DEV)
    got = _native.linear_rows(dx, dw)
    lib = torch.nn.functional.linear(dx, dw)
    torch.cuda.synchronize()
    exact = x.double() @ w.double().T
    got = got.cpu().double()
    err = ((got - exact).abs() - exact.abs() * 2.0**-8).max().item()
    ulp_diff = (got != lib.cpu().double()).double().mean().item()
    _log(f"  excess over half an ulp={err:.3e} differs from torch's GEMM={ulp_diff:.5f}")
    assert err <= 1e-5
    assert ulp_diff < 0.01


@pytest.mark.parametrize("rows", [3, 16])
def test_linear_rows_silu_mul_matches_reference_formula(rows):
    """The SwiGLU epilogue: gate and up from float64 products rounded to bf16,
    then silu rounded and the product rounded (nie_silu_mul's arithmetic),
    against nie_linear_rows with the fused [gate; up] weight; outputs whose
    gate or up landed on the other side of a rounding boundary are the only
    ones allowed to differ (< 1%).  One ulp on gate and on up, carried through
    silu's rounding and the product's, stays within 6 bf16 ulps, so the
    bound is 2^-5 relative (8 ulps); a wrong operand or index gives O(1)."""
    inner, k = 8192, 2048
    _log(f"linear_rows silu_mul rows={rows}")
    x, w = _linear_inputs(rows, 2 * inner, k, seed=11 + rows)
    w = (w.float() * 3).to(torch.bfloat16)  # gate values of a few units, where silu bends
    got = _native.linear_rows(x.to(DEV), w.to(DEV), silu_mul=True)
    torch.cuda.synchronize()
    prod = x.double() @ w.double().T
    gate = prod[:, :inner].to(torch.bfloat16).float()
    up = prod[:, inner:].to(torch.bfloat16).float()
    want = (torch.nn.functional.silu(gate).to(torch.bfloat16).float() * up).to(torch.bfloat16).float()
    got = got.cpu().float()
    assert got.shape == (rows, inner)
    rel = ((got - want).abs() / want.abs().clamp_min(1e-3)).max().item()
    mism = (got != want).float().mean().item()
    _log(f"  max_rel_err={rel:.3e} mismatching={mism:.5f}")
    assert rel <= 2.0**-5
    assert mism < 0.01


def test_linear_rows_rejects_unsupported_shapes_on_the_gpu():
    """17 rows or an in-size that is not a multiple of 2048 raise before any
    launch (callers keep torch's GEMM for them)."""
    x = torch.zeros((17, 2048), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((64, 2048), dtype=torch.bfloat16, device=DEV)
    assert not _native.linear_rows_supported(x, w)
    with pytest.raises(RuntimeError, match="nie_linear_rows"):
        _native.linear_rows(x, w)
    assert not _native.linear_rows_supported(x[:4, :1024], w[:, :1024])
    assert _native.linear_rows_supported(x[:16], w)


@pytest.mark.parametrize("rows", [1, 7, 16])
@pytest.mark.parametrize("with_residual", [False, True])
@pytest.mark.parametrize("silu", [False, True])
def test_rms_norm_linear_rows_matches_norm_then_product(rows, with_residual, silu):
    """nie_rms_norm_linear_rows, each stage against its own bar:
    - the residual sum bit for bit (x + residual in bf16);
    - the folded norm's operand (read back exactly through an identity
      weight) bit for bit equal to nie_rms_norm's output (the kernel reduces
      the sum of squares in rms_norm_kernel's order), and against the
      reference norm formula in fp32 as nie_rms_norm is held: within one
      bf16 ulp, < 1% of elements off;
    - the product against float64 over that operand: half an ulp for the
      plain epilogue, the SwiGLU epilogue as for nie_linear_rows."""
    k, n = 2048, (2 * 4096 if silu else 3072)
    _log(f"rms_norm_linear_rows rows={rows} residual={with_residual} silu={silu}")
    gen = torch.Generator().manual_seed(rows * 100 + with_residual * 10 + silu)
    x = torch.randn((rows, k), generator=gen).to(torch.bfloat16)
    res = torch.randn((rows, k), generator=gen).to(torch.bfloat16) if with_residual else None
    nw = (1 + 0.1 * torch.randn(k, generator=gen)).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=gen) * (3 if silu else 1) / k**0.5).to(torch.bfloat16)
    dx, dnw = x.to(DEV), nw.to(DEV)
    dres = None if res is None else res.to(DEV)
    s_got, got = _native.rms_norm_linear_rows(dx, dres, dnw, 1e-5, w.to(DEV), silu_mul=silu)
    _, xn_k = _native.rms_norm_linear_rows(dx, dres, dnw, 1e-5, torch.eye(k, dtype=torch.bfloat16, device=DEV),
                                           want_sum=False)
    torch.cuda.synchronize()
    h = x + res if res is not None else x
    if res is not None:
        assert torch.equal(s_got.cpu(), h)
    else:
        assert s_got is None
    if dres is not None:
        _, sep_norm = _native.rms_norm(dx, dnw, 1e-5, residual=dres)
    else:
        sep_norm = _native.rms_norm(dx, dnw, 1e-5)
    torch.cuda.synchronize()
    xn_k = xn_k.cpu()
    assert torch.equal(xn_k, sep_norm.cpu())
    xn = _rms_norm_reference(h, nw, 1e-5).float()
    n_rel = ((xn_k.float() - xn).abs() / xn.abs().clamp_min(1e-3)).max().item()
    n_mism = (xn_k.float() != xn).float().mean().item()
    _log(f"  norm operand: max_rel_err={n_rel:.3e} mismatching={n_mism:.5f}")
    assert n_rel <= 2.0**-7 and n_mism < 0.01
    prod = xn_k.double() @ w.double().T
    got = got.cpu().float()
    if silu:
        gate = prod[:, : n // 2].to(torch.bfloat16).float()
        up = prod[:, n // 2:].to(torch.bfloat16).float()
        want = (torch.nn.functional.silu(gate).to(torch.bfloat16).float() * up).to(torch.bfloat16).float()
        rel = ((got - want).abs() / want.abs().clamp_min(1e-3)).max().item()
        mism = (got != want).float().mean().item()
        _log(f"  product: max_rel_err={rel:.3e} mismatching={mism:.5f}")
        assert rel <= 2.0**-5 and mism < 0.01
    else:
        err = ((got.double() - prod).abs() - prod.abs() * 2.0**-8).max().item()
        _log(f"  product: excess over half an ulp={err:.3e}")
        assert err <= 1e-5


def _random_shape(rng):
    """(kv_heads, q_heads, head_dim, block_size, dtype, host_plan) of a sweep case."""
    kv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([g for g in (1, 2, 4, 8, 16) if kv * g <= 64]))
    return (kv, kv * group, int(rng.choice([64, 128])), int(rng.choice([5, 8, 16, 32])),
            torch.bfloat16 if rng.random() < 0.7 else torch.float32, bool(rng.random() < 0.6))


@pytest.mark.parametrize("seed", range(24))
def test_varlen_prefill_random_sweep(seed):
    """Seeded random ragged batches against the oracle: 1-8 requests, contexts
    0-2000, query chunks 1-160 (about a third of the requests single-token),
    1-8 KV heads, GQA groups 1-16, head_dim 64 or 128, block sizes 5-32, fp32
    or bf16, launches planned from host lengths or from bounds."""
    rng = np.random.default_rng(1000 + seed)
    kv, hq, d, bs, dtype, host_plan = _random_shape(rng)
    n = int(rng.integers(1, 9))
    ctx = [int(x) for x in rng.integers(0, 2001, size=n)]
    q = [1 if rng.random() < 0.33 else int(x) for x in rng.integers(1, 161, size=n)]
    _log(f"varlen sweep {seed}: ctx={ctx} q={q} hkv={kv} hq={hq} d={d} bs={bs} {dtype} host_plan={host_plan}")
    wl = workloads.ragged(ctx, q, seed=seed, pool_factor=1.3, q_heads=hq, kv_heads=kv, head_dim=d, block_size=bs)
    got, want = _prefill_case(wl, dtype, host_plan)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("seed", range(24))
def test_decode_random_sweep(seed):
    """Seeded random decode batches against the oracle: 1-24 sequences of
    1-6000 tokens, with the shapes of the prefill sweep."""
    rng = np.random.default_rng(2000 + seed)
    kv, hq, d, bs, dtype, host_plan = _random_shape(rng)
    n = int(rng.integers(1, 25))
    ctx = [int(x) for x in rng.integers(0, 6000, size=n)]
    _log(f"decode sweep {seed}: {n} seqs, max ctx {max(ctx)} hkv={kv} hq={hq} d={d} bs={bs} {dtype} host_plan={host_plan}")
    wl = workloads.ragged(ctx, [1] * n, seed=seed, pool_factor=1.3, q_heads=hq, kv_heads=kv, head_dim=d,
                          block_size=bs)
    kc, vc = wl.pool(dtype)
    qt, _, _ = wl.new_tokens(dtype)
    got = _decode_hip(wl, kc.to(DEV), vc.to(DEV), qt, dtype, host_plan)
    want = _decode_oracle(wl, kc, vc, qt)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_decode_append_device_plan_matches_host_plan(dtype):
    """nie_paged_decode_append_planned, planned from a bucket's bounds and
    reading its work items from a device plan written by write_decode_plan,
    equals nie_paged_decode_append planned from the same host lengths bit for
    bit, cache included; with a zeroed plan it equals the launch planned
    from the bounds."""
    from nano_infer_engine.paged_batch import decode_plan_bound

    _log(f"decode-append device plan {dtype}")
    wl = workloads.ragged([500, 37, 3000, 128, 1999], [1] * 5, seed=41, pool_factor=1.5)
    kc, vc = wl.pool(dtype)
    q, k_new, v_new = wl.new_tokens(dtype)
    host = list(wl.seq_lens)
    bound = decode_plan_bound(max(host))
    tab = wl.table_array()
    width = max(tab.shape[1], -(-bound // wl.block_size))
    padded = np.zeros((tab.shape[0], width), dtype=np.int32)
    padded[:, : tab.shape[1]] = tab
    tables = torch.from_numpy(padded).to(DEV)
    lens = torch.tensor(host, dtype=torch.int32, device=DEV)
    qd, kd, vd = q.to(DEV), k_new.to(DEV), v_new.to(DEV)
    scale = wl.head_dim**-0.5
    plan = np.zeros(_native.decode_plan_bytes() // 4, dtype=np.int32)
    _native.write_decode_plan(plan.ctypes.data, plan.nbytes, dtype, wl.q_heads, wl.kv_heads, wl.head_dim,
                              wl.block_size, np.asarray(host, dtype=np.int32), max(host), sum(host))
    assert plan[0] > 0

    def run(**kw):
        k, v = kc.to(DEV), vc.to(DEV)
        if "device_plan" in kw:
            d = _native.PreparedDecode(k, v, tables, lens, bound, len(host) * bound, wl.q_heads, scale, **kw)
        elif kw.get("seq_lens_host") is not None:
            d = _native.PreparedDecode(k, v, tables, lens, max(host), sum(host), wl.q_heads, scale, **kw)
        else:
            d = _native.PreparedDecode(k, v, tables, lens, bound, len(host) * bound, wl.q_heads, scale)
        out = torch.empty_like(qd)
        d.append_decode(qd, kd, vd, 0, out)
        torch.cuda.synchronize()
        return out.cpu(), k.cpu(), v.cpu()

    planned = run(device_plan=torch.from_numpy(plan.view(np.uint8)).to(DEV))
    host_planned = run(seq_lens_host=host)
    assert all(torch.equal(a, b) for a, b in zip(planned, host_planned))
    zero_plan = run(device_plan=torch.zeros(_native.decode_plan_bytes(), dtype=torch.uint8, device=DEV))
    bound_planned = run()
    assert all(torch.equal(a, b) for a, b in zip(zero_plan, bound_planned))
    ref_k, ref_v = kc.clone(), vc.clone()
    for b, (table, ctx) in enumerate(zip(wl.tables, wl.context_lens)):
        reference_ops.write_tokens(ref_k, ref_v, 0, table, wl.block_size, ctx, k_new[b : b + 1], v_new[b : b + 1])
    want = _decode_oracle(wl, ref_k, ref_v, q)
    err = (planned[0].float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]
