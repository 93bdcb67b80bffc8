"""The paged path above the kernels, on the GPU: cache data movement, the
drop-in attention functions, the model, chunked prefill and the scheduler.

Restates the reference's own tests for these callers
(``tests/test_paged_cache.py:208-315``, ``tests/test_paged_attention.py``,
``tests/test_paged_prefill.py``, ``tests/test_paged_greedy_generation.py``)
with head_dim 64 (the kernels are built for head_dim 64 and 128), and adds
the end-to-end comparison: the same model with its attention core swapped
for the oracle's restatement of the reference algorithm
(``oracle.reference_ops.attention_core_like_product``).
"""

from __future__ import annotations

import contextlib

import pytest
import torch

import nano_infer_engine.layers.attention as attention_module
import nano_infer_engine.layers.linear as linear_module
from nano_infer_engine.generation import (
    ContinuousBatchingScheduler,
    GenerationConfig,
    RequestStatus,
    paged_greedy_generate,
    paged_prefill,
    paged_prefill_chunks,
)
from nano_infer_engine.layers.attention import GroupedQueryAttention
from nano_infer_engine.layers.paged_attention import batched_paged_attention_reference, paged_attention_reference
from nano_infer_engine.models.llama import Llama3_2, LlamaConfig
from nano_infer_engine.paged_cache import PagedKVCache
from oracle import closed_form, reference_ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _log(msg):
    print(msg, flush=True)


@contextlib.contextmanager
def oracle_attention():
    """Run the model with the reference attention algorithm instead of the HIP kernels."""
    saved = attention_module.attention_core
    attention_module.attention_core = reference_ops.attention_core_like_product
    try:
        yield
    finally:
        attention_module.attention_core = saved


@contextlib.contextmanager
def reference_path():
    """The reference's algorithms end to end: the reference attention and
    torch's GEMM for every projection (no nie_linear_rows)."""
    saved = linear_module.USE_NATIVE
    linear_module.USE_NATIVE = False
    try:
        with oracle_attention():
            yield
    finally:
        linear_module.USE_NATIVE = saved


@contextlib.contextmanager
def torch_gemm():
    """The projections on torch's GEMM, attention on the HIP kernels."""
    saved = linear_module.USE_NATIVE
    linear_module.USE_NATIVE = False
    try:
        yield
    finally:
        linear_module.USE_NATIVE = saved


@contextlib.contextmanager
def native_gemm():
    """A decode step's projections on nie_linear_rows (opt-in)."""
    saved = linear_module.USE_NATIVE
    linear_module.USE_NATIVE = True
    try:
        yield
    finally:
        linear_module.USE_NATIVE = saved


def _model(dtype=torch.float32, hidden=256, q_heads=4, kv_heads=2, layers=2, vocab=64, max_seq_len=64, seed=0):
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=vocab, hidden_size=hidden, mlp_inner_size=2 * hidden, num_layers=layers,
                      q_head_num=q_heads, kv_head_num=kv_heads, rope_type="default", max_seq_len=max_seq_len,
                      tie_word_embeddings=False)
    return Llama3_2(cfg).eval().to(DEV, dtype)


def _cache_for(model, num_blocks, block_size=2):
    cfg = model.config
    return PagedKVCache(num_blocks, block_size, cfg.num_layers, cfg.kv_head_num, cfg.head_dim,
                        model.embed.weight.dtype, DEV)


def _cache(num_blocks=6, block_size=4, layers=2, kv=2, d=64, dtype=torch.float32):
    return PagedKVCache(num_blocks, block_size, layers, kv, d, dtype, DEV)


# ---------------------------------------------------------------------------
# PagedKVCache data movement (tests/test_paged_cache.py:208-315)
# ---------------------------------------------------------------------------
def test_gather_of_fragmented_table_is_bit_exact():
    _log("cache gather fragmented")
    cache = _cache()
    for sid in ("temporary-a", "temporary-b", "temporary-c"):
        cache.ensure_capacity(sid, 1)
    cache.release("temporary-a")
    cache.release("temporary-c")
    cache.ensure_capacity("request-a", 6)
    assert cache.get_block_table("request-a") == (2, 0)
    keys = torch.arange(6 * 2 * 64, dtype=torch.float32, device=DEV).reshape(6, 2, 64)
    values = keys + 100
    cache.write(1, "request-a", 0, keys, values)
    gk, gv = cache.gather(1, "request-a", 6)
    assert torch.equal(gk, keys) and torch.equal(gv, values)
    assert torch.equal(cache.keys[1, 2], keys[:4]) and torch.equal(cache.keys[1, 0, :2], keys[4:])


def test_export_import_preserves_kv_and_length():
    _log("cache export/import")
    src, dst = _cache(), _cache()
    src.ensure_capacity("temporary-a", 1)
    src.ensure_capacity("temporary-b", 1)
    src.release("temporary-a")
    dst.ensure_capacity("temporary", 1)
    src.ensure_capacity("request-a", 6)
    expected = []
    for layer in range(2):
        keys = torch.arange(6 * 2 * 64, dtype=torch.float32, device=DEV).reshape(6, 2, 64) + layer * 100
        src.write(layer, "request-a", 0, keys, keys + 1000)
        expected.append((keys, keys + 1000))
    src.advance("request-a", 6)
    transfer = src.export_sequence("request-a")
    dst.import_sequence("request-a", transfer)
    assert dst.get_sequence_length("request-a") == 6
    assert dst.get_block_table("request-a") != src.get_block_table("request-a")
    for layer, (k, v) in enumerate(expected):
        gk, gv = dst.gather(layer, "request-a", 6)
        assert torch.equal(gk, k) and torch.equal(gv, v)


def test_export_is_an_independent_snapshot_with_zero_tail():
    _log("cache export snapshot")
    src = _cache(num_blocks=2, layers=1)
    src.ensure_capacity("request-a", 8)
    keys = torch.ones(2, 2, 64, device=DEV)
    src.write(0, "request-a", 0, keys, keys + 1)
    src.advance("request-a", 2)
    transfer = src.export_sequence("request-a")
    src.keys.zero_()
    src.values.zero_()
    assert torch.equal(transfer.keys[:, :, :2], keys[None, None])
    assert torch.equal(transfer.values[:, :, :2], (keys + 1)[None, None])
    assert transfer.keys.shape[1] == 1
    assert torch.count_nonzero(transfer.keys[:, :, 2:]) == 0 and torch.count_nonzero(transfer.values[:, :, 2:]) == 0


def test_import_rolls_back_when_a_step_fails(monkeypatch):
    _log("cache import rollback")
    src, dst = _cache(num_blocks=2), _cache(num_blocks=2)
    src.ensure_capacity("request-a", 1)
    ones = torch.ones(1, 2, 64, device=DEV)
    src.write(0, "request-a", 0, ones, ones)
    src.advance("request-a", 1)
    transfer = src.export_sequence("request-a")

    def fail(sequence_id, token_count):
        raise RuntimeError("simulated import failure")

    monkeypatch.setattr(dst, "advance", fail)
    with pytest.raises(RuntimeError, match="simulated import failure"):
        dst.import_sequence("request-a", transfer)
    assert dst.allocator.allocated_block_count == 0
    with pytest.raises(KeyError, match="request-a"):
        dst.get_block_table("request-a")


# ---------------------------------------------------------------------------
# drop-in attention functions (tests/test_paged_attention.py)
# ---------------------------------------------------------------------------
def test_paged_attention_reference_matches_contiguous_attention():
    _log("paged_attention_reference layout (3, 0, 2)")
    torch.manual_seed(0)
    q = torch.randn(4, 64)
    ks, vs = torch.randn(5, 2, 64), torch.randn(5, 2, 64)
    kc, vc = torch.randn(2, 4, 2, 2, 64), torch.randn(2, 4, 2, 2, 64)
    reference_ops.write_tokens(kc, vc, 1, (3, 0, 2), 2, 0, ks, vs)
    got = paged_attention_reference(q.to(DEV), kc.to(DEV), vc.to(DEV), (3, 0, 2), 5, 1)
    exact = closed_form.decode(q.numpy(), ks.numpy(), vs.numpy(), 64**-0.5)
    assert (got.cpu() - torch.from_numpy(exact).float()).abs().max().item() <= 1e-4


def test_batched_paged_attention_matches_per_sequence():
    _log("batched paged attention")
    torch.manual_seed(1)
    q = torch.randn(3, 4, 64, device=DEV)
    kc = torch.randn(2, 7, 2, 2, 64, device=DEV)
    vc = torch.randn_like(kc)
    tables = ((5, 1), (4, 0, 6), (2,))
    lengths = (3, 5, 2)
    got = batched_paged_attention_reference(q, kc, vc, tables, lengths, 1)
    each = torch.stack([paged_attention_reference(q[b], kc, vc, tables[b], lengths[b], 1) for b in range(3)])
    assert got.shape == q.shape
    torch.testing.assert_close(got, each, rtol=0, atol=1e-6)
    want = reference_ops.batched_paged_attention_reference(q.cpu(), kc.cpu(), vc.cpu(), tables, lengths, 1)
    assert (got.cpu() - want).abs().max().item() <= 1e-4


def test_paged_attention_validation_messages():
    kc = torch.zeros(1, 2, 2, 2, 64, device=DEV)
    q = torch.zeros(4, 64, device=DEV)
    with pytest.raises(ValueError, match="block_table does not cover sequence_length"):
        paged_attention_reference(q, kc, kc, (0,), 3, 0)
    with pytest.raises(ValueError, match="block ID out of range"):
        paged_attention_reference(q, kc, kc, (0, 2), 3, 0)
    with pytest.raises(IndexError, match="layer_index out of range"):
        paged_attention_reference(q, kc, kc, (0, 1), 3, 1)


def test_gqa_batched_paged_decode_matches_individual_calls():
    _log("GroupedQueryAttention batched decode")
    torch.manual_seed(2)
    attn = GroupedQueryAttention(q_head_num=4, kv_head_num=2, hidden_size=256).eval().to(DEV)
    ids, lengths = ("request-a", "request-b"), (2, 4)
    hist_k = (torch.randn(2, 2, 64, device=DEV), torch.randn(4, 2, 64, device=DEV))
    hist_v = (torch.randn(2, 2, 64, device=DEV), torch.randn(4, 2, 64, device=DEV))

    def build(selected):
        blocks = sum((lengths[ids.index(s)] + 2) // 2 for s in selected)
        cache = PagedKVCache(blocks, 2, 1, 2, 64, torch.float32, DEV)
        for s in selected:
            i = ids.index(s)
            cache.ensure_capacity(s, lengths[i] + 1)
            cache.write(0, s, 0, hist_k[i], hist_v[i])
            cache.advance(s, lengths[i])
        return cache

    x = torch.randn(2, 1, 256, device=DEV)
    with torch.inference_mode():
        got = attn(x, paged_cache=build(ids), layer_index=0, sequence_ids=ids)
        want = torch.cat([attn(x[b : b + 1], paged_cache=build((s,)), layer_index=0, sequence_id=s)
                          for b, s in enumerate(ids)])
    assert got.shape == x.shape
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# model, prefill, chunked prefill
# ---------------------------------------------------------------------------
def test_model_matches_oracle_attention_fp32():
    _log("model vs oracle attention fp32")
    model = _model()
    prompt = torch.tensor([[1, 5, 9, 13, 17, 21, 25, 29, 33, 2, 4]], device=DEV)

    def run():
        cache = _cache_for(model, 16, block_size=4)
        out = [model(prompt, kv_cache=cache)]
        token = prompt[:, -1:]
        for _ in range(4):
            logits = model(token, kv_cache=cache)
            out.append(logits)
            token = logits[:, -1].argmax(-1, keepdim=True)
        return out

    with torch.inference_mode():
        hip = run()
        with oracle_attention():
            ref = run()
    err = max((a - b).abs().max().item() for a, b in zip(hip, ref))
    _log(f"  max_abs_err={err:.3e}")
    assert err <= 1e-4


def test_paged_prefill_matches_individual_prompts():
    _log("paged_prefill vs individual")
    model = _model()
    cache = _cache_for(model, 8)
    prompts = (torch.tensor([[1, 4]], device=DEV), torch.tensor([[1, 5, 8, 11]], device=DEV))
    with torch.inference_mode():
        want = torch.cat([model(p)[:, -1] for p in prompts])
        got = paged_prefill(model, prompts, cache, ("request-a", "request-b"))
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    assert cache.get_sequence_length("request-a") == 2 and cache.get_sequence_length("request-b") == 4
    assert set(cache.get_block_table("request-a")).isdisjoint(cache.get_block_table("request-b"))


def test_chunked_prefill_matches_one_shot():
    _log("chunked == one-shot")
    model = _model()
    prompt = torch.tensor([[1, 4, 7, 10, 13, 3, 8, 5, 30]], device=DEV)
    one, chunked = _cache_for(model, 8), _cache_for(model, 8)
    with torch.inference_mode():
        want = paged_prefill(model, (prompt,), one, ("request-a",))
        for lo, hi in ((0, 2), (2, 5), (5, 9)):
            got = paged_prefill_chunks(model, (prompt[:, lo:hi],), chunked, ("request-a",))
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    assert chunked.get_sequence_length("request-a") == 9
    for layer in range(2):
        a = one.gather(layer, "request-a", 9)
        b = chunked.gather(layer, "request-a", 9)
        torch.testing.assert_close(a[0], b[0], rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(a[1], b[1], rtol=1e-5, atol=1e-5)


def test_ragged_chunks_in_one_call_match_separate_calls():
    _log("ragged tails together == separately")
    model = _model()
    prompts = {"request-a": torch.tensor([[1, 4, 7, 10, 13]], device=DEV),
               "request-b": torch.tensor([[2, 6, 3]], device=DEV)}
    together, apart = _cache_for(model, 12), _cache_for(model, 12)
    with torch.inference_mode():
        for cache in (together, apart):
            paged_prefill_chunks(model, (prompts["request-a"][:, :2], prompts["request-b"][:, :1]), cache,
                                 ("request-a", "request-b"))
        got = paged_prefill_chunks(model, (prompts["request-a"][:, 2:], prompts["request-b"][:, 1:]), together,
                                   ("request-a", "request-b"))
        want = torch.cat([
            paged_prefill_chunks(model, (prompts["request-a"][:, 2:],), apart, ("request-a",)),
            paged_prefill_chunks(model, (prompts["request-b"][:, 1:],), apart, ("request-b",)),
        ])
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# scheduler with a real model
# ---------------------------------------------------------------------------
def test_scheduler_known_answers_with_real_model():
    _log("scheduler known answers (real model)")
    model = _model(max_seq_len=16)
    cache = _cache_for(model, 8, block_size=1)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=1, prefill_chunk_size=2), cache, 1)
    a = s.add_request("request-a", torch.tensor([[1, 2, 3, 4, 5]], device=DEV))
    for offset in (2, 4):
        assert s.step().token_events == ()
        assert a.status is RequestStatus.PREFILLING and a.prefill_offset == offset
        assert cache.get_sequence_length("request-a") == offset

    cache = _cache_for(model, 24, block_size=1)
    s = ContinuousBatchingScheduler(
        model, GenerationConfig(max_new_tokens=1, prefill_chunk_size=2, max_prefill_tokens_per_step=3), cache, 3
    )
    reqs = [s.add_request(f"request-{i}", torch.tensor([[1, 2, 3, 4, 5, 6]], device=DEV)) for i in range(3)]
    for offsets in ((2, 1, 0), (3, 1, 2), (3, 3, 3)):
        s.step()
        assert tuple(r.prefill_offset for r in reqs) == offsets

    cache = _cache_for(model, 12, block_size=1)
    s = ContinuousBatchingScheduler(model, GenerationConfig(max_new_tokens=2, prefill_chunk_size=2), cache, 2)
    ra = s.add_request("request-a", torch.tensor([[1]], device=DEV))
    rb = s.add_request("request-b", torch.tensor([[2, 3, 4, 5]], device=DEV))
    calls = []
    original = model.forward_ragged

    def recording(input_ids, *, kv_cache, sequence_ids, query_start_loc):
        calls.append((tuple(sequence_ids), tuple(query_start_loc.tolist())))
        return original(input_ids, kv_cache=kv_cache, sequence_ids=sequence_ids, query_start_loc=query_start_loc)

    model.forward_ragged = recording
    try:
        s.step()
        assert ra.status is RequestStatus.ACTIVE and rb.status is RequestStatus.PREFILLING
        calls.clear()
        out = s.step()
    finally:
        del model.forward_ragged
    assert calls == [(("request-b", "request-a"), (0, 2, 3))]
    assert out.token_events[0].sequence_id == "request-a"


def test_greedy_tokens_identical_to_oracle_attention_fp32():
    _log("greedy identity fp32")
    model = _model(vocab=128, max_seq_len=128)
    prompts = tuple(torch.randint(0, 128, (1, n), generator=torch.Generator().manual_seed(n)).to(DEV)
                    for n in (3, 17, 40))
    cfg = GenerationConfig(max_new_tokens=24, prefill_chunk_size=8, max_prefill_tokens_per_step=16)

    def run():
        cache = _cache_for(model, 64, block_size=4)
        return paged_greedy_generate(model, prompts, cfg, cache, ("a", "b", "c"))

    hip = run()
    with oracle_attention():
        ref = run()
    for x, y in zip(hip.sequences, ref.sequences):
        assert torch.equal(x, y)


def test_bf16_teacher_forced_matches_oracle_attention():
    """bf16 Llama-shaped heads (32 q / 8 kv, head_dim 64): logits of a prefill
    and 24 teacher-forced decode steps, HIP (attention kernels and the decode
    steps' projection GEMMs) vs the reference algorithm (reference attention,
    torch's GEMMs).

    The two differ by bf16 rounding order only: max abs logit error <= 5e-2.
    The top-1 token must match on every row whose reference top-2 margin is
    larger than twice the observed error (no error of that size can reorder
    them), such rows must be the majority, and on the others the HIP pick must
    be one of the reference's near-top tokens.  A random-init model has exact
    bf16 ties and one-ulp margins on a few rows, where both picks are correct
    argmaxes of logits equal to within rounding."""
    _log("bf16 teacher forced")
    model = _model(dtype=torch.bfloat16, hidden=2048, q_heads=32, kv_heads=8, layers=2, vocab=512, max_seq_len=512)
    for p in model.parameters():
        if p.ndim > 1:
            torch.nn.init.normal_(p, 0.0, 0.02)
    gen = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 512, (1, 200), generator=gen).to(DEV)
    follow = torch.randint(0, 512, (24,), generator=gen).tolist()

    def run():
        cache = _cache_for(model, 32, block_size=16)
        rows = [model(prompt, kv_cache=cache)[0, -1]]
        for t in follow:
            rows.append(model(torch.tensor([[t]], device=DEV), kv_cache=cache)[0, -1])
        return torch.stack(rows).float()

    with torch.inference_mode():
        hip = run()
        with reference_path():
            ref = run()
    err = (hip - ref).abs().max().item()
    top2 = ref.topk(2, dim=-1).values
    decisive = (top2[:, 0] - top2[:, 1]) > 2 * err
    agree = (hip.argmax(-1) == ref.argmax(-1)).float().mean().item()
    _log(f"  logits max_abs_err={err:.3e} top1 agreement={agree:.3f} decisive rows={int(decisive.sum())}/{len(ref)}")
    assert err <= 5e-2
    assert decisive.float().mean().item() >= 0.5
    assert torch.equal(hip.argmax(-1)[decisive], ref.argmax(-1)[decisive])
    picked = ref.gather(1, hip.argmax(-1, keepdim=True)).squeeze(1)
    assert bool((top2[:, 0] - picked <= 2 * err).all())


def test_bf16_batched_decode_projections_match_torch_gemm():
    """16 sequences through two Llama-3.2-1B-shaped blocks (hidden 2048, 32 q /
    8 kv heads, SwiGLU 4096, vocab 32768, bf16): prefill, then 6 decode steps
    of 16 rows each, whose projections, gated product and LM head run on
    nie_linear_rows, against the same steps on torch's GEMM (the attention
    kernels the same in both).  The two differ by accumulation order only:
    max abs logit error <= 5e-2, top-1 identical on rows whose margin exceeds
    twice that error (the majority)."""
    _log("bf16 batched decode projections")
    model = _model(dtype=torch.bfloat16, hidden=2048, q_heads=32, kv_heads=8, layers=2, vocab=32768,
                   max_seq_len=128)
    for p in model.parameters():
        if p.ndim > 1:
            torch.nn.init.normal_(p, 0.0, 0.02)
    gen = torch.Generator().manual_seed(4)
    prompt = torch.randint(0, 32768, (16, 24), generator=gen).to(DEV)
    follow = torch.randint(0, 32768, (16, 6), generator=gen).to(DEV)

    ids = tuple(f"seq-{i}" for i in range(16))

    def run():
        cache = _cache_for(model, 16 * 3, block_size=16)
        rows = [model(prompt, kv_cache=cache, sequence_ids=ids)[:, -1]]
        for t in range(follow.shape[1]):
            rows.append(model(follow[:, t:t + 1], kv_cache=cache, sequence_ids=ids)[:, -1])
        return torch.cat(rows).float()

    with torch.inference_mode():
        with native_gemm():
            hip = run()
        with torch_gemm():
            ref = run()
    err = (hip[16:] - ref[16:]).abs().max().item()
    assert torch.equal(hip[:16], ref[:16])  # the prefill rows take torch's GEMM in both runs
    top2 = ref.topk(2, dim=-1).values
    decisive = (top2[:, 0] - top2[:, 1]) > 2 * err
    _log(f"  decode logits max_abs_err={err:.3e} decisive rows={int(decisive.sum())}/{len(ref)}")
    assert 0 < err <= 5e-2
    assert decisive.float().mean().item() >= 0.5
    assert torch.equal(hip.argmax(-1)[decisive], ref.argmax(-1)[decisive])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lean_prefill_blocks_match_generic_blocks(monkeypatch, dtype):
    """A packed forward of more than 16 rows (two prefill chunks on cached
    context plus a decode row) runs each block through forward_tokens_lean:
    the norms, SiLU product and attention on this library's kernels, the
    projections on torch's GEMM with stacked [q; k; v] and [gate; up]
    weights.  The same call through the generic blocks (which stack the same
    weights and call the same kernels through the module layer) gives the
    same logits and cache bit for bit."""
    _log(f"lean prefill blocks == generic blocks ({dtype})")
    from nano_infer_engine.layers.decoder import Llama3Decoder
    model = _model(dtype=dtype, hidden=512, q_heads=8, kv_heads=2, layers=3, vocab=256, max_seq_len=128, seed=6)
    gen = torch.Generator().manual_seed(6)
    ids = ("request-a", "request-b", "request-c")
    prompts = [torch.randint(0, 256, (1, n), generator=gen).to(DEV) for n in (40, 21, 9)]
    lengths = (24, 31, 1)
    flat = torch.randint(0, 256, (sum(lengths),), generator=gen).to(DEV)
    bounds = torch.tensor([0, 24, 55, 56], device=DEV)

    lean_calls = []
    original = Llama3Decoder.forward_tokens_lean

    def spy(self, *args, **kwargs):
        lean_calls.append(1)
        return original(self, *args, **kwargs)

    monkeypatch.setattr(Llama3Decoder, "forward_tokens_lean", spy)

    def run():
        cache = _cache_for(model, 24, block_size=8)
        with torch.inference_mode():
            for p, sid in zip(prompts, ids):
                model(p, kv_cache=cache, sequence_ids=(sid,))
            lean_calls.clear()
            logits = model.forward_ragged(flat, kv_cache=cache, sequence_ids=ids, query_start_loc=bounds)
        torch.cuda.synchronize()
        return logits, cache

    lean_logits, lean_cache = run()
    assert len(lean_calls) == model.config.num_layers
    with monkeypatch.context() as m:
        m.setattr(Llama3_2, "_lean_stream", lambda self, x: None)
        generic_logits, generic_cache = run()
    assert not lean_calls
    assert torch.equal(lean_logits, generic_logits)
    for sid in ids:
        n = lean_cache.get_sequence_length(sid)
        assert n == generic_cache.get_sequence_length(sid)
        for layer in range(model.config.num_layers):
            lk, lv = lean_cache.gather(layer, sid, n)
            gk, gv = generic_cache.gather(layer, sid, n)
            assert torch.equal(lk, gk) and torch.equal(lv, gv)


def test_lean_prefill_blocks_follow_weight_changes(monkeypatch):
    """The lean blocks' cached weights follow the parameters: after an
    in-place change of one projection and after a projection's weight is
    replaced, a 40-row forward gives the generic blocks' logits bit for bit,
    and different logits than before the change."""
    _log("lean prefill blocks follow weight changes")
    model = _model(dtype=torch.bfloat16, hidden=512, q_heads=8, kv_heads=2, layers=2, vocab=256, max_seq_len=64, seed=8)
    prompt = torch.randint(0, 256, (1, 40), generator=torch.Generator().manual_seed(8)).to(DEV)

    def run(lean):
        with monkeypatch.context() as m:
            if not lean:
                m.setattr(Llama3_2, "_lean_stream", lambda self, x: None)
            cache = _cache_for(model, 8, block_size=8)
            with torch.inference_mode():
                out = model(prompt, kv_cache=cache, sequence_ids=("s",))
            torch.cuda.synchronize()
            return out

    before = run(True)
    with torch.no_grad():
        model.decoders[1].attn.o_proj.weight.mul_(1.5)
    changed = run(True)
    assert torch.equal(changed, run(False)) and not torch.equal(changed, before)
    down = model.decoders[0].ffn.down_proj
    down.weight = torch.nn.Parameter(down.weight.detach() * 0.5)
    replaced = run(True)
    assert torch.equal(replaced, run(False)) and not torch.equal(replaced, changed)
