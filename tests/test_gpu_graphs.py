"""On-device greedy argmax and HIP-graph replay of the decode step.

* ``argmax_rows`` == ``torch.argmax(dim=-1)`` (ties to the lowest index,
  NaN largest), bit for bit.
* A replayed decode step (``DecodeGraphRunner``) computes exactly what the
  eager step computes on an identical cache: same logits bits, same next
  tokens, same cache contents — across replays with eager work and
  synchronisations between them, a batch-size change and a crossing of the
  decode plan's length bucket (both of which capture a new graph).
* The scheduler produces the same tokens with and without decode graphs.
"""

from __future__ import annotations

import pytest
import torch

from nano_infer_engine import _native
from nano_infer_engine.generation import ContinuousBatchingScheduler, GenerationConfig, paged_prefill, paged_prefill_chunks
from nano_infer_engine.generation.decode_graph import DecodeGraphRunner
from nano_infer_engine.models.llama import Llama3_2, LlamaConfig
from nano_infer_engine.paged_cache import PagedKVCache

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_rows_matches_torch(dtype):
    _log(f"argmax_rows {dtype}")
    gen = torch.Generator(device=DEV).manual_seed(3)
    wide = torch.randn((9, 1031), generator=gen, device=DEV).to(dtype)
    logits = wide[:, 1:1026]  # rows start off 16-byte alignment
    logits[2, 17] = logits[2, 900] = 50.0  # a tie: the lower index wins
    logits[3] = 1.0  # all equal: index 0
    logits[4, 333] = float("nan")  # NaN is the largest
    logits[5, 1024] = 60.0  # the last element
    got = _native.argmax_rows(logits)
    assert torch.equal(got, logits.argmax(dim=-1))
    aligned = torch.randn((16, 128256), generator=gen, device=DEV).to(dtype)
    # the vector path loads 8 vectors per thread at once: a tie across those
    # batches, the row's last element, NaN, an all-equal row
    aligned[0, 5] = aligned[0, 128000] = 100.0
    aligned[1, 128255] = 100.0
    aligned[2, 64000] = float("nan")
    aligned[3] = 1.0
    aligned[6, 8191] = aligned[6, 8192] = 100.0  # a tie across two pieces of the split form
    aligned[7, 128255] = float("inf")
    assert torch.equal(_native.argmax_rows(aligned), aligned.argmax(dim=-1))  # split form (>= 2 pieces)
    # the split form on rows that start off 16-byte alignment and a short last piece
    wide2 = torch.randn((5, 8192 * 3 + 11), generator=gen, device=DEV).to(dtype)
    odd = wide2[:, 1:]
    odd[1, 8192 * 2 + 5] = 100.0
    assert torch.equal(_native.argmax_rows(odd), odd.argmax(dim=-1))
    short = torch.randn((3, 8192), generator=gen, device=DEV).to(dtype)  # one-workgroup form
    assert torch.equal(_native.argmax_rows(short), short.argmax(dim=-1))


def _graph_model(dtype):
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=512, hidden_size=256, mlp_inner_size=512, num_layers=2, q_head_num=4,
                      kv_head_num=2, rope_type="llama3", max_seq_len=2048, tie_word_embeddings=False)
    return Llama3_2(cfg).eval().to(DEV, dtype)


def _cache(model, num_blocks=256):
    cfg = model.config
    return PagedKVCache(num_blocks, 16, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, model.embed.weight.dtype, DEV)


@pytest.mark.parametrize("dtype,max_graphs", [(torch.float32, 64), (torch.bfloat16, 64), (torch.bfloat16, 1)])
def test_decode_graph_replays_match_eager_step(dtype, max_graphs):
    """Replays equal eager steps; captures share one memory pool, and with
    max_graphs=1 every new (batch, bucket) key evicts the previous capture.
    Odd steps pass the token IDs as a host list (they travel with the
    metadata copy), even steps as the device tensor."""
    _log(f"decode graph vs eager {dtype} max_graphs={max_graphs}")
    model = _graph_model(dtype)
    gen = torch.Generator(device=DEV).manual_seed(1)
    # the first prompt crosses the 512-token plan bucket during the decode steps
    prompts = [torch.randint(0, 512, (1, n), generator=gen, device=DEV) for n in (500, 37, 300)]
    ids = ("a", "b", "c")
    graph_cache, eager_cache = _cache(model), _cache(model)
    with torch.inference_mode():
        first = paged_prefill(model, tuple(prompts), graph_cache, ids)
        assert torch.equal(first, paged_prefill(model, tuple(prompts), eager_cache, ids))
    runner = DecodeGraphRunner(model, graph_cache, max_batch_size=4, max_graphs=max_graphs)
    tokens = first.argmax(dim=-1)
    active = list(ids)
    for step in range(24):
        if step == 14:  # one sequence leaves: a new batch size
            active, tokens = active[:2], tokens[:2]
        with torch.inference_mode():
            if step % 2:
                g_logits, g_next = runner.step(None, tuple(active), host_ids=tokens.tolist())
            else:
                g_logits, g_next = runner.step(tokens, tuple(active))
            g_logits, g_next = g_logits.clone(), g_next.clone()
            e_logits = paged_prefill_chunks(model, tuple(t.view(1, 1) for t in tokens), eager_cache, tuple(active))
        if step % 5 == 0:
            torch.cuda.synchronize()
        assert torch.equal(g_logits, e_logits), f"step {step}: logits differ"
        assert torch.equal(g_next, e_logits.argmax(dim=-1)), f"step {step}: next tokens differ"
        tokens = g_next
    for sid in ids:  # the sequences' cached tokens (unused pool slots hold whatever the allocation held)
        n = graph_cache.get_sequence_length(sid)
        assert n == eager_cache.get_sequence_length(sid)
        assert graph_cache.get_block_table(sid) == eager_cache.get_block_table(sid)
        for layer in range(model.config.num_layers):
            gk, gv = graph_cache.gather(layer, sid, n)
            ek, ev = eager_cache.gather(layer, sid, n)
            assert torch.equal(gk, ek) and torch.equal(gv, ev)
    assert graph_cache.get_sequence_length("a") > 512  # the bucket was crossed
    assert runner.captures == 3 and runner.replays == 24
    assert runner.evictions == (0 if max_graphs >= 3 else 2)
    _log(f"  captures={runner.captures} replays={runner.replays} evictions={runner.evictions}")


def test_decode_graph_logits_survive_other_captures():
    """A step's logits (and next IDs) stay as they were while other captures
    replay: two batch sizes (two captures sharing one memory pool) are
    replayed alternately, and each step's returned logits, read back after
    the other capture's next replay, still hold what they held when
    returned."""
    _log("decode graph logits across captures")
    model = _graph_model(torch.bfloat16)
    gen = torch.Generator(device=DEV).manual_seed(2)
    prompts = [torch.randint(0, 512, (1, n), generator=gen, device=DEV) for n in (40, 90, 17, 64, 33)]
    ids = ("a", "b", "c", "d", "e")
    cache = _cache(model)
    with torch.inference_mode():
        first = paged_prefill(model, tuple(prompts), cache, ids)
    runner = DecodeGraphRunner(model, cache, max_batch_size=8)
    tokens = {sid: first[i].argmax(-1).view(1) for i, sid in enumerate(ids)}
    groups = (("a", "b"), ("c", "d", "e"))
    held = []  # (logits view, next view, copies at return time)
    for step in range(6):
        group = groups[step % 2]
        with torch.inference_mode():
            logits, nxt = runner.step(torch.cat([tokens[s] for s in group]), group)
        torch.cuda.synchronize()
        held.append((logits, nxt, logits.clone(), nxt.clone()))
        for i, s in enumerate(group):
            tokens[s] = nxt[i].view(1).clone()
        if step >= 1:  # the previous step (the other capture) was returned before this replay
            old_logits, old_next, want_logits, want_next = held[step - 1]
            assert torch.equal(old_logits, want_logits) and torch.equal(old_next, want_next), step
    assert runner.captures == 2 and runner.replays == 6


def test_scheduler_tokens_identical_with_decode_graphs():
    _log("scheduler with decode graphs")
    model = _graph_model(torch.bfloat16)
    gen = torch.Generator(device=DEV).manual_seed(2)
    prompts = [torch.randint(0, 512, (1, n), generator=gen, device=DEV) for n in (40, 7, 90, 33, 64, 21)]
    runs = []
    for graphs in (False, True):
        cache = _cache(model)
        config = GenerationConfig(max_new_tokens=24, eos_token_id=None, prefill_chunk_size=16,
                                  max_prefill_tokens_per_step=32)
        sched = ContinuousBatchingScheduler(model, config, cache, max_batch_size=4, decode_graphs=graphs)
        reqs = [sched.add_request(f"r{i}", p) for i, p in enumerate(prompts)]
        sched.run_until_idle()
        runs.append([r.sequence.clone() for r in reqs])
        if graphs:
            assert sched._graphs.replays > 0
            _log(f"  graph captures={sched._graphs.captures} replays={sched._graphs.replays}")
            # completed requests keep their own last logits
            assert all(r.last_logits is not None for r in reqs)
    for a, b in zip(*runs):
        assert torch.equal(a, b)
