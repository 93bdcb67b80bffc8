"""Shapes the MFMA kernels are not built for run on the generic attention kernel.

head_dim outside {64, 128} (the reference's own tests use 1, 3 and 4) and
GQA groups outside {1, 2, 4, 8, 16}: decode, varlen prefill, the fused
append (+ RoPE) decode step and the RoPE append, through the same C ABI
entry points.  Bars as for the tuned kernels: attention fp32 max-abs <= 1e-4
and bf16 <= 2e-2 against the oracle, caches bit-exact, the fused calls
bit-identical to the separate ones.
"""

from __future__ import annotations

import pytest
import torch

from nano_infer_engine import _native, workloads
from nano_infer_engine.layers.paged_attention import paged_attention_reference
from oracle import reference_ops
from tests.test_gpu_kernels import TOL, _append_decode_pair, _decode_hip, _decode_oracle, _prefill_case

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

SHAPES = [  # (q_heads, kv_heads, head_dim, block_size)
    (4, 2, 3, 2),
    (4, 2, 4, 1),
    (3, 1, 1, 4),
    (6, 2, 32, 3),  # group 3
    (5, 1, 80, 16),  # group 5
    (12, 4, 96, 16),
    (8, 8, 256, 16),
    (32, 8, 48, 16),
]


def _log(msg: str) -> None:
    print(msg, flush=True)


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,block_size", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generic_decode_matches_oracle(q_heads, kv_heads, head_dim, block_size, dtype):
    _log(f"generic decode hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype}")
    assert not _native.tuned_attention(q_heads, kv_heads, head_dim)
    wl = workloads.ragged([0, 5, 40, 300], [1, 1, 1, 1], seed=41, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    kc, vc = wl.pool(dtype)
    q, _, _ = wl.new_tokens(dtype)
    got = _decode_hip(wl, kc.to(DEV), vc.to(DEV), q, dtype, host_plan=True)
    want = _decode_oracle(wl, kc, vc, q)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,block_size", SHAPES[:6])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generic_varlen_prefill_matches_oracle(q_heads, kv_heads, head_dim, block_size, dtype):
    _log(f"generic prefill hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} {dtype}")
    wl = workloads.ragged([0, 3, 50, 0, 17], [19, 5, 1, 40, 2], seed=43, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    got, want = _prefill_case(wl, dtype)
    err = (got.float() - want.float()).abs().max().item()
    _log(f"  max_abs_err={err:.3e}")
    assert err <= TOL[dtype]


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,block_size", [(6, 2, 32, 3), (5, 1, 80, 16), (4, 2, 4, 1)])
@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generic_decode_append_matches_separate_calls(q_heads, kv_heads, head_dim, block_size, rope, dtype):
    """The fused step on a generic shape (append kernel, then attention that
    rotates q itself) equals the append (or RoPE append) then decode, and
    the oracle."""
    _log(f"generic decode_append hq={q_heads} hkv={kv_heads} d={head_dim} bs={block_size} rope={rope} {dtype}")
    wl = workloads.ragged([0, 4, 15, 16, 70, 300], [1] * 6, seed=47, pool_factor=1.5, q_heads=q_heads,
                          kv_heads=kv_heads, head_dim=head_dim, block_size=block_size)
    _append_decode_pair(wl, dtype, True, layer=1, rope=rope)


@pytest.mark.parametrize("head_dim", [2, 32, 80])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_generic_rope_kv_append_bit_exact(head_dim, dtype):
    from nano_infer_engine.layers.rope import RopeScale

    _log(f"generic rope_kv_append d={head_dim} {dtype}")
    q_heads, kv_heads = 6, 2
    gen = torch.Generator(device=DEV).manual_seed(53)
    tokens, num_blocks, bs, layers, layer = 29, 48, 4, 2, 1
    qkv = torch.randn((tokens, q_heads + 2 * kv_heads, head_dim), generator=gen, device=DEV).to(dtype)
    q, k, v = qkv[:, :q_heads], qkv[:, q_heads : q_heads + kv_heads], qkv[:, q_heads + kv_heads :]
    positions = torch.randint(0, 4000, (tokens,), generator=gen, device=DEV, dtype=torch.int64)
    slots = torch.randperm(num_blocks * bs, generator=gen, device=DEV)[:tokens].to(torch.int64)
    slots[3] = -1
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
    cos, sin = rope.tables(DEV, dtype, 4000)
    _native.rope_kv_append(kc, vc, layer, q, k, v, positions, slots, cos, sin)
    torch.cuda.synchronize()
    assert torch.equal(q, q_want)
    assert torch.equal(kc, kc_want) and torch.equal(vc, vc_want)


def test_reference_paged_attention_test_shape():
    """tests/test_paged_attention.py:11-56 of the reference, on the GPU: head_dim
    3, 4 query / 2 KV heads, a fragmented table; the paged result equals
    softmax attention over the contiguous keys (GQA map h -> h // 2)."""
    torch.manual_seed(0)
    q_heads, kv_heads, head_dim, block_size, length = 4, 2, 3, 2, 5
    query = torch.randn(q_heads, head_dim)
    keys = torch.randn(length, kv_heads, head_dim)
    values = torch.randn(length, kv_heads, head_dim)
    key_cache = torch.randn(2, 4, block_size, kv_heads, head_dim)
    value_cache = torch.randn(2, 4, block_size, kv_heads, head_dim)
    table = (3, 1, 0)
    for pos in range(length):
        block, off = table[pos // block_size], pos % block_size
        key_cache[1, block, off] = keys[pos]
        value_cache[1, block, off] = values[pos]
    got = paged_attention_reference(query.to(DEV), key_cache.to(DEV), value_cache.to(DEV), table, length, 1).cpu()
    k_rep = keys.repeat_interleave(q_heads // kv_heads, dim=1)
    v_rep = values.repeat_interleave(q_heads // kv_heads, dim=1)
    scores = torch.einsum("hd,thd->ht", query, k_rep) * head_dim**-0.5
    want = torch.einsum("ht,thd->hd", torch.softmax(scores, dim=-1), v_rep)
    torch.testing.assert_close(got, want)
