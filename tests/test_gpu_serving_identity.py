"""End-to-end serving numerics of the Llama-3.2-1B-shaped model against the reference path (bf16 and fp32).

The product runs as shipped: the continuous-batching scheduler with chunked
prefill (chunk 128, 512 prefill tokens per step, batch 16, block size 16),
decode steps replayed from HIP graphs, the library's decode-step GEMMs; 16
requests with prompts of 128..2048 tokens, 256 greedy tokens each, bf16,
random N(0, 0.02) weights.  After every step the same forward is replayed
(teacher-forced) on the reference algorithm in bf16, in fp32 (the truth,
same weights), and in a bf16 variant with fp32 attention products
(``oracle.lockstep``).

What the measurements show on this random-init model: both bf16 paths carry
~0.12 of max-abs logit error against the fp32 truth, and top-2 margins are
often a few bf16 ulps, so two bf16 implementations that differ only in
accumulation order — the reference and its variant — already diverge
within a few dozen tokens.  Identical 256-token greedy output is therefore
a property of bit-identical arithmetic only.  The bar here is that the
product is as faithful to the fp32 truth as the reference path: the same
top-1 agreement with the truth (within 1 point) and the same logit error
(median within 5%, p99 within 10%); and every row where the product and the
reference pick different tokens is a near-tie whose reference margin is
covered by the measured difference of the two rows.
"""

from __future__ import annotations

import json

import pytest
import torch

from nano_infer_engine import workloads
from nano_infer_engine.paged_cache import PagedKVCache
from oracle import lockstep

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def test_serving_tokens_against_reference_path():
    print("serving lockstep: llama-1b shape, 16 requests x 256 tokens, chunk 128 / 512, batch 16", flush=True)
    model = workloads.serving_model(DEV)
    cfg = model.config
    prompts = workloads.serving_prompts(DEV, cfg.vocab_size, count=16)
    blocks = workloads.serving_cache_blocks(prompts, 256)

    def cache(dtype):
        return PagedKVCache(blocks, 16, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, dtype, DEV)

    report = lockstep.run_lockstep(model, prompts, cache, max_new_tokens=256, max_batch_size=16, chunk=128,
                                   budget=512, variant=True)
    s = report.summary()
    print(json.dumps({k: v for k, v in s.items() if k != "first_divergence"}), flush=True)
    print("first divergence tokens:", sorted(v["token"] for v in s["first_divergence"].values() if v), flush=True)
    assert s["requests"] == 16 and s["sampled_rows"] == 16 * 256
    assert all(seq.shape[1] == p.shape[1] + 256 for seq, p in zip(report.sequences.values(), prompts))
    # as faithful to the fp32 truth as the reference path
    assert s["top1_agreement_product_truth"] >= s["top1_agreement_reference_truth"] - 0.01
    assert s["err_product_truth"]["median"] <= 1.05 * s["err_reference_truth"]["median"]
    assert s["err_product_truth"]["p99"] <= 1.10 * s["err_reference_truth"]["p99"]
    # every disagreement is a near-tie inside the measured row difference
    for row in report.rows:
        if row.product != row.reference:
            assert row.reference_margin <= 2 * row.err_product_reference, row


def test_serving_tokens_against_reference_path_fp32():
    """The same serving run in fp32 (the bf16 model's weights upcast): the
    product's greedy tokens equal the reference path's.  Teacher forcing with
    every sampled row agreeing is free-running identity, by induction over
    the steps.  Logit error here is ~1e-5, so only an exact tie could flip a
    row; any flip must be such a near-tie."""
    print("serving lockstep fp32: llama-1b shape, 16 requests x 256 tokens, chunk 128 / 512, batch 16", flush=True)
    model = workloads.serving_model(DEV).float()
    cfg = model.config
    prompts = workloads.serving_prompts(DEV, cfg.vocab_size, count=16)
    blocks = workloads.serving_cache_blocks(prompts, 256)

    def cache(dtype):
        return PagedKVCache(blocks, 16, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, dtype, DEV)

    report = lockstep.run_lockstep(model, prompts, cache, max_new_tokens=256, max_batch_size=16, chunk=128,
                                   budget=512, truth=False)
    s = report.summary()
    print(json.dumps({k: v for k, v in s.items() if k != "first_divergence"}), flush=True)
    assert s["requests"] == 16 and s["sampled_rows"] == 16 * 256
    assert s["err_product_reference"]["max"] <= 1e-3
    assert s["top1_agreement_product_reference"] >= 0.999
    for row in report.rows:
        if row.product != row.reference:
            assert row.reference_margin <= 2 * row.err_product_reference, row
