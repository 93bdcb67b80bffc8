"""Long-context decode through the whole Llama-3.2-1B-shaped model (16 x 29,600 tokens).

The product serves 16 sequences of 29,600 cached tokens with captured decode
steps (``DecodeGraphRunner``: the fused RoPE + append + attention launch of
every layer, replayed from a HIP graph) over a 16-layer paged cache whose
allocator hands out a seeded random permutation of its 40,000 blocks, so
the tables are scattered over the whole pool and every layer past the third
sits beyond 2**31 elements of its K / V tensor.  The cached contexts are
N(0, 1) values, the same in the reference's cache (identical tables and
contents).  After 8 greedy steps of the product, the same 8 steps are
replayed teacher-forced on the reference algorithm (``ReferenceLlama``:
``models/llama.py:339-394``, ``layers/attention.py:345-414``) and compared
row by row:

* fp32 (the bf16 model's weights upcast): identical argmaxes and logits
  within 1e-4;
* bf16: as close to the reference as the reference's own fp32-product
  variant is (the serving bar of ``test_gpu_serving_identity``, scaled for
  128 rows): median logit error within 25% of the variant's, top-1
  agreement within five points of the variant's.

Pool sizing follows ``service/runtime.py:128-154`` in spirit (a pool far
larger than the working set, blocks from anywhere in it); the attention-only
16 x 29,600 step on a 300,000-block pool is ``test_gpu_long_context``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_infer_engine import workloads
from nano_infer_engine.generation.decode_graph import DecodeGraphRunner
from nano_infer_engine.paged_cache import PagedKVCache
from oracle.reference_model import ReferenceLlama

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
CTX, STEPS, SEQS, POOL_BLOCKS, BS = 29600, 8, 16, 40_000, 16


def _log(msg: str) -> None:
    print(msg, flush=True)


def _cache(cfg, dtype, seed_perm: int) -> PagedKVCache:
    """A cache whose free list is a seeded permutation of the whole pool,
    with the 16 sequences' blocks reserved and CTX tokens marked cached."""
    cache = PagedKVCache(POOL_BLOCKS, BS, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, dtype, DEV)
    everything = cache.allocator.allocate(POOL_BLOCKS)
    cache.allocator.free(np.random.default_rng(seed_perm).permutation(everything).tolist())
    for sid in _ids():
        cache.ensure_capacity(sid, CTX + STEPS + 1)
        cache.advance(sid, CTX)
    return cache


def _ids() -> tuple[str, ...]:
    return tuple(f"long-{i}" for i in range(SEQS))


def _fill(cache: PagedKVCache) -> None:
    """N(0, 1) K/V in every block the sequences hold, every layer."""
    used = torch.tensor(sorted(b for sid in _ids() for b in cache.get_block_table(sid)), device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(4)
    shape = (used.numel(), BS, cache.kv_head_num, cache.head_dim)
    for layer in range(cache.num_layers):
        for pool in (cache.keys, cache.values):
            pool[layer, used] = torch.randn(shape, generator=gen, device=DEV).to(pool.dtype)


def _twin(cache: PagedKVCache, seed_perm: int) -> PagedKVCache:
    """A second cache with the same tables and contents."""
    cfg = type("Cfg", (), {"num_layers": cache.num_layers, "kv_head_num": cache.kv_head_num,
                           "head_dim": cache.head_dim})
    other = _cache(cfg, cache.keys.dtype, seed_perm)
    for sid in _ids():
        assert other.get_block_table(sid) == cache.get_block_table(sid)
    other.keys.copy_(cache.keys)
    other.values.copy_(cache.values)
    return other


def _serve(model, cache):
    """8 greedy captured decode steps: per step the input tokens and the logits."""
    runner = DecodeGraphRunner(model, cache, SEQS)
    gen = torch.Generator(device=DEV).manual_seed(9)
    tokens = torch.randint(0, model.config.vocab_size, (SEQS,), generator=gen, device=DEV)
    inputs, logits = [], []
    for step in range(STEPS):
        inputs.append(tokens.clone())
        out, tokens = runner.step(tokens, _ids())
        logits.append(out.float().clone())  # static buffers: copy before the next replay
        torch.cuda.synchronize()
        _log(f"  product step {step}")
    assert runner.captures >= 1 and runner.replays == STEPS
    return inputs, logits


def _replay(ref: ReferenceLlama, cache, inputs):
    """The same steps, teacher-forced, on the reference algorithm."""
    out = []
    starts = torch.arange(SEQS + 1, dtype=torch.int64)
    for step, tokens in enumerate(inputs):
        out.append(ref.forward_ragged(tokens, kv_cache=cache, sequence_ids=_ids(), query_start_loc=starts).float())
        torch.cuda.synchronize()
        _log(f"  reference step {step}")
    return out


def _assert_positions(cache, expected: int) -> None:
    for sid in _ids():
        assert cache.get_sequence_length(sid) == expected


def test_long_context_model_fp32_matches_reference():
    _log(f"long-context model fp32: {SEQS} x {CTX} tokens, {POOL_BLOCKS}-block shuffled pool, {STEPS} graph steps")
    model = workloads.serving_model(DEV).to(torch.float32)
    cfg = model.config
    cache = _cache(cfg, torch.float32, seed_perm=5)
    assert (cfg.num_layers - 1) * cache.keys[0].numel() > 2**31  # late layers' offsets exceed 2**31
    _fill(cache)
    ref_cache = _twin(cache, seed_perm=5)
    inputs, got = _serve(model, cache)
    want = _replay(ReferenceLlama(model), ref_cache, inputs)
    _assert_positions(cache, CTX + STEPS)
    _assert_positions(ref_cache, CTX + STEPS)
    worst = 0.0
    for step, (a, b) in enumerate(zip(got, want)):
        err = (a - b).abs().max().item()
        worst = max(worst, err)
        same = torch.equal(a.argmax(-1), b.argmax(-1))
        _log(f"  step {step}: max |logit diff| {err:.2e}, argmax identical {same}")
        assert same, step
    assert worst <= 1e-4, worst
    # the appended K/V rows (RoPE'd keys, values) agree with the reference's writes
    for sid in _ids():
        table = np.asarray(cache.get_block_table(sid), dtype=np.int64)
        pos = np.arange(CTX, CTX + STEPS)
        slots = torch.from_numpy(table[pos // BS] * BS + pos % BS).to(DEV)
        for layer in (0, cfg.num_layers - 1):
            for mine, theirs in ((cache.keys, ref_cache.keys), (cache.values, ref_cache.values)):
                a = mine[layer].view(-1, cfg.kv_head_num, cfg.head_dim)[slots]
                b = theirs[layer].view(-1, cfg.kv_head_num, cfg.head_dim)[slots]
                assert (a - b).abs().max().item() <= 1e-4


def test_long_context_model_bf16_within_variant_bar():
    _log(f"long-context model bf16: {SEQS} x {CTX} tokens, {POOL_BLOCKS}-block shuffled pool, {STEPS} graph steps")
    model = workloads.serving_model(DEV)
    cfg = model.config
    cache = _cache(cfg, torch.bfloat16, seed_perm=6)
    _fill(cache)
    ref_cache = _twin(cache, seed_perm=6)
    var_cache = _twin(cache, seed_perm=6)
    inputs, got = _serve(model, cache)
    want = _replay(ReferenceLlama(model), ref_cache, inputs)
    var = _replay(ReferenceLlama(model, fp32_attention_products=True), var_cache, inputs)
    _assert_positions(cache, CTX + STEPS)
    g, w, v = torch.cat(got), torch.cat(want), torch.cat(var)
    err_product = (g - w).abs().amax(-1)
    err_variant = (v - w).abs().amax(-1)
    top1_product = (g.argmax(-1) == w.argmax(-1)).float().mean().item()
    top1_variant = (v.argmax(-1) == w.argmax(-1)).float().mean().item()
    _log(f"  rows {g.shape[0]}: top-1 agreement product {top1_product:.4f} variant {top1_variant:.4f}; "
         f"median logit error product {err_product.median().item():.4f} variant {err_variant.median().item():.4f}")
    assert top1_product >= top1_variant - 0.05
    assert err_product.median().item() <= 1.25 * err_variant.median().item()
