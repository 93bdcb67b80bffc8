"""Benchmark of the paged-attention decode path on one MI355X.

Workload (one "step"): a continuous-batching decode step of the Llama-3.2-1B
attention geometry — 16 ragged sequences with lognormal context lengths
(median 2048, sigma 1, clipped to [32, 29600], seed 1), 32 query / 8 KV
heads, head_dim 64, block_size 16, bf16, block tables drawn from a seeded
permutation of a pool twice the size needed.  For each of the 16 layers the
step appends one new K/V token per sequence through ``slot_mapping`` and runs
paged decode attention over the grown sequences.  16 layers give a 1.4 GB
working set, far beyond the 256 MB last-level cache, so every step reads
its KV from HBM.

Prints one JSON line.  ``value`` = algorithmic bytes (decode K/V/Q/O/table
reads + append traffic) per second over the timed steps.  ``roofline`` is
for the decode-attention op, timed per launch with HIP events on its
stream.  ``cpu_baseline`` times the oracle's restatement of the reference
PyTorch algorithm on the host cores over a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "nano-infer-engine_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=40)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=16)
    p.add_argument("--skip-cpu", action="store_true", help="do not time the CPU baseline")
    p.add_argument("--unfused-append", action="store_true",
                   help="decode step as nie_kv_append then nie_paged_decode (two launches per layer)")
    p.add_argument("--skip-stress", action="store_true", help="do not run the 16x29600 decode figure")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="target duration of the CPU sample")
    p.add_argument("--skip-mixed", action="store_true", help="do not run the mixed chunked-prefill figure")
    p.add_argument("--skip-e2e", action="store_true", help="do not run the end-to-end serving figure")
    p.add_argument("--e2e-only", action="store_true", help="run only the end-to-end serving figure")
    p.add_argument("--e2e-ref-steps", type=int, default=3,
                   help="scheduler steps timed with the reference attention algorithm")
    p.add_argument("--mixed-only", action="store_true", help="run only the mixed chunked-prefill figure")
    p.add_argument("--linear-only", action="store_true",
                   help="run only the decode-step projection GEMM figure (nie_linear_rows vs torch's GEMM)")
    p.add_argument("--stress-only", action="store_true",
                   help="run only the 16x29600 decode figure (for per-workload profiles)")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run 4 device-to-device copies of MIB MiB (reference for HBM byte counters)")
    return p.parse_args()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


class DecodeBench:
    """Device state for repeated append+decode steps over one workload."""

    def __init__(self, wl, steps_total: int, device, seed: int):
        import numpy as np
        import torch

        self.wl = wl
        self.device = device
        bs = wl.block_size
        # extend every table so it holds the tokens appended by all steps
        rng = np.random.default_rng(seed + 500)
        need = [-(-(c + steps_total + 1) // bs) for c in wl.context_lens]
        self.num_blocks = max(int(sum(need) * 2), wl.num_blocks)
        perm = rng.permutation(self.num_blocks)
        tables, cursor = [], 0
        for n in need:
            tables.append(perm[cursor : cursor + n])
            cursor += n
        width = max(len(t) for t in tables)
        table_arr = np.zeros((len(tables), width), dtype=np.int32)
        for r, t in enumerate(tables):
            table_arr[r, : len(t)] = t
        shape = (wl.num_layers, self.num_blocks, bs, wl.kv_heads, wl.head_dim)
        gen = torch.Generator(device=device).manual_seed(seed)
        self.k_cache = torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16)
        self.v_cache = torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16)
        self.tables = torch.from_numpy(table_arr).to(device)
        b = len(tables)
        # per-step metadata, built before any timing
        slots = np.zeros((steps_total, b), dtype=np.int64)
        lens = np.zeros((steps_total, b), dtype=np.int32)
        self.max_len, self.total_len, self.seq_lens_host = [], [], []
        for s in range(steps_total):
            pos = np.asarray(wl.context_lens) + s
            slots[s] = table_arr[np.arange(b), pos // bs].astype(np.int64) * bs + pos % bs
            lens[s] = pos + 1
            self.max_len.append(int(lens[s].max()))
            self.total_len.append(int(lens[s].sum()))
            self.seq_lens_host.append(lens[s].tolist())
        self.slots = torch.from_numpy(slots).to(device)
        self.lens = torch.from_numpy(lens).to(device)
        self.q = torch.randn((b, wl.q_heads, wl.head_dim), generator=gen, device=device, dtype=torch.bfloat16)
        self.k_new = torch.randn((b, wl.kv_heads, wl.head_dim), generator=gen, device=device, dtype=torch.bfloat16)
        self.v_new = torch.randn_like(self.k_new)
        self.out = torch.empty_like(self.q)
        self.scale = wl.head_dim**-0.5

    def step(self, s: int, events: list | None = None, fused: bool = True) -> None:
        """One decode step over every layer; optionally brackets each decode launch with HIP events.

        fused: one ``nie_paged_decode_append`` launch per layer writes the new
        token and attends; otherwise ``nie_kv_append`` then ``nie_paged_decode``
        (the events then bracket the decode call only).  The launches are
        prepared once per step and reused by every layer, as a model forward
        does (``RaggedBatch.launchers``).
        """
        import torch

        from nano_infer_engine import _native

        append = None if fused else _native.PreparedAppend(self.k_cache, self.v_cache, self.slots[s])
        decode = _native.PreparedDecode(self.k_cache, self.v_cache, self.tables, self.lens[s], self.max_len[s],
                                        self.total_len[s], self.wl.q_heads, self.scale,
                                        seq_lens_host=self.seq_lens_host[s])
        for layer in range(self.wl.num_layers):
            if append is not None:
                append(self.k_new, self.v_new, layer)
            if events is not None:
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record()
            if append is None:
                decode.append_decode(self.q, self.k_new, self.v_new, layer, self.out)
            else:
                decode(self.q, layer, self.out)
            if events is not None:
                end.record()
                events.append((start, end))


def run_gpu(args):
    import torch

    from nano_infer_engine import _native, workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    _native.load_library()
    wl = workloads.decode_ragged(num_layers=args.layers)
    # steps [0, W) warm up, [W, W+K) are the timed steps, [W+K, W+2K) are
    # timed again per call with HIP events (kept out of the wall-clock pass,
    # whose host and queue work they would add to)
    timed_end = args.warmup + args.steps
    total_steps = timed_end + args.steps
    bench = DecodeBench(wl, total_steps, device, seed=1)
    log(f"workload: {len(wl.context_lens)} seqs, contexts {wl.context_lens}, layers {args.layers}, "
        f"pool {bench.num_blocks} blocks ({2 * bench.k_cache.numel() * 2 / 1e9:.2f} GB)")

    fused = not args.unfused_append
    for s in range(args.warmup):
        bench.step(s, fused=fused)
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    for s in range(args.warmup, timed_end):
        bench.step(s, fused=fused)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    ev: list = []
    for s in range(timed_end, total_steps):
        bench.step(s, ev, fused=fused)
    torch.cuda.synchronize()

    step_append = workloads.append_bytes(len(wl.context_lens))
    decode_bytes = sum(workloads.decode_bytes(bench.seq_lens_host[s]) for s in range(args.warmup, timed_end))
    decode_bytes *= args.layers
    append_bytes = step_append * args.layers * args.steps
    event_bytes = sum(workloads.decode_bytes(bench.seq_lens_host[s]) for s in range(timed_end, total_steps))
    launch_ms = [a.elapsed_time(b) for a, b in ev]
    avg_launch_s = sum(launch_ms) / len(launch_ms) / 1e3
    # a fused call also moves the appended rows
    bytes_per_launch = event_bytes * args.layers / len(launch_ms) + (step_append if fused else 0)
    achieved = bytes_per_launch / avg_launch_s / 1e9
    value = (decode_bytes + append_bytes) / elapsed / 1e9
    call = "nie_paged_decode_append" if fused else "nie_paged_decode"
    log(f"timed {args.steps} steps in {elapsed * 1e3:.2f} ms ({value:.0f} GB/s); {call} call avg "
        f"{avg_launch_s * 1e6:.2f} us for {bytes_per_launch / 1e6:.2f} MB -> {achieved:.0f} GB/s")

    result = {
        "metric": "paged-attn HBM GB/s (% of peak); e2e output tok/s, Llama-1B-shape batch 16",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) K/V/Q, seeded lognormal context lengths",
        "config": {
            "workload": "continuous-batching decode step: 16 ragged sequences (lognormal median 2048, "
                        "sigma 1, clip [32, 29600], seed 1), 32 q / 8 kv heads, head_dim 64, block_size 16, "
                        f"append 1 token/seq then paged decode attention, x{args.layers} layers"
                        + (" (one fused launch per layer)" if fused else " (separate append launch)"),
            "sequences": len(wl.context_lens),
            "context_tokens_first_step": int(sum(wl.context_lens)),
            "layers": args.layers,
            "global_batch": len(wl.context_lens),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"{call} call: paged_decode_kernel + decode_merge_kernel (HIP events around the call)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _measured_traffic(),
            "algorithmic_bytes_per_launch": int(bytes_per_launch),
            "avg_launch_us": round(avg_launch_s * 1e6, 3),
        },
    }
    del bench
    torch.cuda.empty_cache()
    if not args.skip_stress:
        result["stress_16x29600"] = run_stress(args)
    if not args.skip_mixed:
        result["mixed_prefill_step"] = run_mixed(args)
    if not args.skip_e2e:
        result["e2e_llama1b_serving"] = run_e2e(args)
    return result


def run_stress(args):
    """Decode over 16 x 29600-token contexts (970 MB per layer-step), one layer."""
    import torch

    from nano_infer_engine import workloads

    device = torch.device("cuda:0")
    steps, warmup = 20, 3
    wl = workloads.decode_long(num_layers=1)
    bench = DecodeBench(wl, steps + warmup, device, seed=4)
    fused = not args.unfused_append
    for s in range(warmup):
        bench.step(s, fused=fused)
    torch.cuda.synchronize()
    ev: list = []
    for s in range(warmup, warmup + steps):
        bench.step(s, ev, fused=fused)
    torch.cuda.synchronize()
    launch_ms = [a.elapsed_time(b) for a, b in ev]
    avg = sum(launch_ms) / len(launch_ms) / 1e3
    per_launch = sum(workloads.decode_bytes(bench.seq_lens_host[s]) for s in range(warmup, warmup + steps)) / steps
    if fused:
        per_launch += workloads.append_bytes(len(wl.context_lens))
    gbs = per_launch / avg / 1e9
    log(f"stress 16x29600: {avg * 1e6:.1f} us per layer-step, {gbs:.0f} GB/s")
    del bench
    torch.cuda.empty_cache()
    return {"avg_launch_us": round(avg * 1e6, 2), "bytes_per_launch": int(per_launch),
            "achieved_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def run_mixed(args):
    """Mixed chunked-prefill step: 4 x 128-token chunks on contexts {0, 384, 1024, 4000}
    + 12 decode rows (contexts U[256, 8192]), packed varlen layout, one layer.

    Times the varlen prefill launch (algorithmic FLOPs over unmasked pairs vs
    the bf16 MFMA peak) and the decode launch of the same step separately.
    """
    import numpy as np
    import torch

    from nano_infer_engine import _native, workloads

    device = torch.device("cuda:0")
    wl = workloads.mixed_prefill()
    kc, vc = wl.pool(torch.bfloat16, device)
    q, k_new, v_new = wl.new_tokens(torch.bfloat16, device)
    slots = torch.from_numpy(wl.slots()).to(device)
    _native.kv_append(kc, vc, 0, k_new, v_new, slots)
    n_pref = 4
    pref_tokens = int(sum(wl.query_lens[:n_pref]))
    tables = torch.from_numpy(wl.table_array()).to(device)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(wl.query_lens[:n_pref])]), dtype=torch.int64, device=device)
    ctx = torch.tensor(wl.context_lens[:n_pref], dtype=torch.int32, device=device)
    seq_lens = wl.seq_lens
    dec_lens = torch.tensor(seq_lens[n_pref:], dtype=torch.int32, device=device)
    scale = wl.head_dim ** -0.5
    prefill = _native.PreparedPrefill(kc, vc, cu, ctx, tables[:n_pref].contiguous(), pref_tokens,
                                      max(wl.query_lens[:n_pref]), max(seq_lens[:n_pref]), wl.q_heads, scale,
                                      cu_seqlens_host=cu.cpu().tolist(), context_lens_host=wl.context_lens[:n_pref])
    decode = _native.PreparedDecode(kc, vc, tables[n_pref:].contiguous(), dec_lens, max(seq_lens[n_pref:]),
                                    sum(seq_lens[n_pref:]), wl.q_heads, scale, seq_lens_host=seq_lens[n_pref:])
    out = torch.empty_like(q)
    qp, op = q[:pref_tokens], out[:pref_tokens]
    qd, od = q[pref_tokens:], out[pref_tokens:]
    reps, warm = 50, 5
    for _ in range(warm):
        prefill(qp, 0, op)
        decode(qd, 0, od)
    torch.cuda.synchronize()
    pev, dev_ = [], []
    for _ in range(reps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        prefill(qp, 0, op)
        e[1].record()
        decode(qd, 0, od)
        e[2].record()
        pev.append((e[0], e[1]))
        dev_.append((e[1], e[2]))
    torch.cuda.synchronize()
    # medians: an event pair also spans the host's launch of the call, so a
    # host stall (a page fault, the garbage collector) would skew a mean
    p_us = float(np.median([a.elapsed_time(b) for a, b in pev])) * 1e3
    d_us = float(np.median([a.elapsed_time(b) for a, b in dev_])) * 1e3
    flops = workloads.prefill_flops(wl.context_lens[:n_pref], wl.query_lens[:n_pref])
    tflops = flops / (p_us * 1e-6) / 1e12
    dbytes = workloads.decode_bytes(seq_lens[n_pref:])
    gbs = dbytes / (d_us * 1e-6) / 1e9
    log(f"mixed step: prefill {p_us:.1f} us = {tflops:.1f} TFLOP/s ({flops / 1e9:.2f} GFLOP); "
        f"decode rows {d_us:.1f} us = {gbs:.0f} GB/s")
    del kc, vc
    torch.cuda.empty_cache()
    return {
        "prefill": {"kernel": "varlen_prefill_kernel", "avg_launch_us": round(p_us, 2), "flops_per_launch": flops,
                    "achieved_TFLOPs": round(tflops, 2), "peak_TFLOPs": MFMA_BF16_PEAK_TFLOPS,
                    "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "decode_rows": {"avg_launch_us": round(d_us, 2), "bytes_per_launch": dbytes, "achieved_GBs": round(gbs, 1),
                        "frac": round(gbs / HBM_PEAK_GBS, 4)},
    }


E2E_REQUESTS = 64
E2E_NEW_TOKENS = 256


def build_e2e_model(device):
    """Llama-3.2-1B shape (LlamaConfig defaults), bf16, Linear/Embedding weights N(0, 0.02), norms 1."""
    import torch
    from torch import nn

    from nano_infer_engine.models.llama import Llama3_2, LlamaConfig

    torch.manual_seed(3)
    with torch.device(device):
        model = Llama3_2(LlamaConfig())
    model = model.to(torch.bfloat16).eval()
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, 0.02)
    return model


def e2e_prompts(device, vocab, count=E2E_REQUESTS, seed=3):
    import numpy as np
    import torch

    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 2049, size=count)
    return [torch.from_numpy(rng.integers(0, vocab, size=(1, int(n)))).to(device) for n in lens]


def e2e_run(model, prompts, device, max_new_tokens, max_steps=None, graphs=True):
    """Serve every prompt through the continuous-batching scheduler; returns (seconds, steps, requests).

    With ``graphs`` the all-decode steps replay captured HIP graphs (captures
    happen inside the timed region, as in a fresh server)."""
    import torch

    from nano_infer_engine.generation import ContinuousBatchingScheduler, GenerationConfig
    from nano_infer_engine.paged_cache import PagedKVCache

    cfg = model.config
    blocks_per_request = -(-(max(p.shape[1] for p in prompts) + max_new_tokens) // 16)
    cache = PagedKVCache(16 * blocks_per_request + 64, 16, cfg.num_layers, cfg.kv_head_num, cfg.head_dim,
                         torch.bfloat16, device)
    gen = GenerationConfig(max_new_tokens=max_new_tokens, eos_token_id=None, prefill_chunk_size=128,
                           max_prefill_tokens_per_step=512)
    sched = ContinuousBatchingScheduler(model, gen, cache, max_batch_size=16, decode_graphs=graphs)
    reqs = [sched.add_request(f"request-{i}", p) for i, p in enumerate(prompts)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    steps = 0
    while sched.has_work and (max_steps is None or steps < max_steps):
        sched.step()
        steps += 1
    torch.cuda.synchronize()
    return time.perf_counter() - t0, steps, reqs


def run_e2e(args):
    """Configuration-4 serving run, and the same model with the reference attention algorithm."""
    import torch

    import nano_infer_engine.layers.attention as attention_module
    from oracle import reference_ops

    device = torch.device("cuda:0")
    model = build_e2e_model(device)
    prompts = e2e_prompts(device, model.config.vocab_size)
    e2e_run(model, prompts[:2], device, 8)  # warm-up: library load, GEMM heuristics
    secs, steps, reqs = e2e_run(model, prompts, device, E2E_NEW_TOKENS)
    out_tokens = sum(r.generated_tokens for r in reqs)
    tok_s = out_tokens / secs
    log(f"e2e: {out_tokens} output tokens from {len(prompts)} requests in {secs:.2f} s "
        f"({steps} steps) -> {tok_s:.0f} tok/s")
    eager_secs, _, eager_reqs = e2e_run(model, prompts, device, E2E_NEW_TOKENS, graphs=False)
    eager_tok_s = sum(r.generated_tokens for r in eager_reqs) / eager_secs
    same_modes = all(torch.equal(a.sequence, b.sequence) for a, b in zip(reqs, eager_reqs))
    log(f"e2e eager (no decode graphs): {eager_secs:.2f} s -> {eager_tok_s:.0f} tok/s; "
        f"tokens identical to the graph run: {same_modes}")
    # the reference attention algorithm (per-request gather / repeat_interleave /
    # matmul / mask / softmax) under the same scheduler, on the first steps only
    k = args.e2e_ref_steps
    ours_k, _, ours_reqs = e2e_run(model, prompts, device, E2E_NEW_TOKENS, max_steps=k)
    # the reference's algorithms end to end: its attention loop and torch's
    # GEMM for every projection
    import nano_infer_engine.layers.linear as linear_module

    saved = attention_module.attention_core
    saved_native = linear_module.USE_NATIVE
    attention_module.attention_core = reference_ops.attention_core_like_product
    linear_module.USE_NATIVE = False
    try:
        ref_k, _, ref_reqs = e2e_run(model, prompts, device, E2E_NEW_TOKENS, max_steps=k)
    finally:
        attention_module.attention_core = saved
        linear_module.USE_NATIVE = saved_native
    same = all(torch.equal(a.sequence, b.sequence) for a, b in zip(ours_reqs, ref_reqs))
    log(f"e2e first {k} steps: ours {ours_k * 1e3:.1f} ms, reference algorithms {ref_k * 1e3:.1f} ms "
        f"({ref_k / ours_k:.1f}x); sequences identical: {same}")
    del model
    torch.cuda.empty_cache()
    return {
        "output_tok_per_s": round(tok_s, 1),
        "output_tok_per_s_eager": round(eager_tok_s, 1),
        "eager_tokens_identical": same_modes,
        "output_tokens": out_tokens,
        "seconds": round(secs, 3),
        "scheduler_steps": steps,
        "workload": "Llama-3.2-1B shape, bf16, random N(0, 0.02) weights; 64 requests, prompts U[128, 2048] "
                    "(seed 3), 256 greedy tokens each, max batch 16, prefill chunk 128, 512 prefill tokens/step",
        "reference_first_steps": {"steps": k, "ours_ms": round(ours_k * 1e3, 2), "reference_ms": round(ref_k * 1e3, 2),
                                  "speedup": round(ref_k / ours_k, 2), "sequences_identical": same},
    }


def run_linear(args):
    """Decode-step projections of the Llama-3.2-1B shape at 16 rows, bf16:
    nie_linear_rows against torch's GEMM (F.linear, hipBLASLt), each timed
    over 20 calls replayed from a captured HIP graph (launch overhead out),
    the calls rotating over weight copies that together exceed the 256 MB
    last-level cache.  Bytes = the weight (2 n k); the gate/up row is the
    fused SwiGLU epilogue against F.linear + nie_silu_mul."""
    import torch
    import torch.nn.functional as F

    from nano_infer_engine import _native

    device = torch.device("cuda:0")
    shapes = [("q/k/v", 3072, 2048, False), ("o_proj", 2048, 2048, False),
              ("gate/up + SiLU", 16384, 2048, True), ("down", 2048, 8192, False),
              ("LM head", 128256, 2048, False)]
    calls = 20
    out = {}
    for name, n, k, glu in shapes:
        copies = max(2, min(calls, int(1.5e9 // (n * k * 2))))
        gen = torch.Generator(device=device).manual_seed(n)
        ws = [torch.randn((n, k), generator=gen, device=device).to(torch.bfloat16) for _ in range(copies)]
        x = torch.randn((16, k), generator=gen, device=device).to(torch.bfloat16)

        def ours(i):
            return _native.linear_rows(x, ws[i % copies], silu_mul=glu)

        def lib(i):
            y = F.linear(x, ws[i % copies])
            if glu:
                g, u = y.split((n // 2, n // 2), dim=-1)
                return _native.silu_mul(g, u)
            return y

        res = {}
        for tag, fn in (("nie_linear_rows", ours), ("torch", lib)):
            for i in range(3):
                fn(i)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(calls):
                    fn(i)
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            e0.record()
            for _ in range(reps):
                graph.replay()
            e1.record()
            torch.cuda.synchronize()
            res[tag] = e0.elapsed_time(e1) * 1e3 / (reps * calls)
            del graph
        gbs = n * k * 2 / (res["nie_linear_rows"] * 1e-6) / 1e9
        out[name] = {"n": n, "k": k, "us": round(res["nie_linear_rows"], 2), "GBs": round(gbs, 1),
                     "frac": round(gbs / 8000.0, 4), "torch_us": round(res["torch"], 2)}
        log(f"{name:15s} {n}x{k}: nie_linear_rows {res['nie_linear_rows']:.2f} us ({gbs:.0f} GB/s), "
            f"torch {res['torch']:.2f} us")
        del ws
        torch.cuda.empty_cache()
    return out


def _measured_traffic():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if present."""
    path = os.path.join(REPO, "profiles", "paged_decode_kernel__decode_step_b16_lognormal__hbm_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def run_cpu_baseline(args):
    """The oracle (reference algorithm, torch on CPU) on a bounded sample of the workload."""
    import torch

    from nano_infer_engine import workloads
    from oracle import reference_ops

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    wl = workloads.decode_ragged(num_layers=1)
    kc, vc = wl.pool(torch.bfloat16)
    q, _, _ = wl.new_tokens(torch.bfloat16)
    tables = tuple(tuple(t) for t in wl.tables)
    lens = tuple(wl.seq_lens)
    reference_ops.batched_paged_attention_reference(q, kc, vc, tables, lens, 0)  # warm-up
    done, t0 = 0, time.perf_counter()
    while True:
        reference_ops.batched_paged_attention_reference(q, kc, vc, tables, lens, 0)
        done += 1
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    elapsed = time.perf_counter() - t0
    gbs = workloads.decode_bytes(lens) * done / elapsed / 1e9
    log(f"cpu baseline: {done} layer-steps in {elapsed:.1f} s on {threads} threads -> {gbs:.3f} GB/s")
    return {
        "value": round(gbs, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} single-layer decode attention calls over the same 16 sequences "
                  f"({sum(lens)} tokens), reference per-block loop in torch bf16 on CPU, {elapsed:.1f} s",
    }


def run_copy_calibration(mib: int):
    """A plain copy of known size: each launch reads and writes mib MiB."""
    import torch

    n = mib * (1 << 20)
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": n, "launches": 4}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the path runs on a single MI355X).", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        run_copy_calibration(args.copy_calibration)
        return
    if args.e2e_only:
        from nano_infer_engine import _native

        _native.load_library()
        print(json.dumps({"e2e_llama1b_serving": run_e2e(args)}), flush=True)
        return
    if args.mixed_only:
        from nano_infer_engine import _native

        _native.load_library()
        print(json.dumps({"mixed_prefill_step": run_mixed(args)}), flush=True)
        return
    if args.linear_only:
        from nano_infer_engine import _native

        _native.load_library()
        print(json.dumps({"decode_projections": run_linear(args)}), flush=True)
        return
    if args.stress_only:
        from nano_infer_engine import _native

        _native.load_library()
        print(json.dumps({"stress_16x29600": run_stress(args)}), flush=True)
        return
    result = run_gpu(args)
    result["cpu_baseline"] = None if args.skip_cpu else run_cpu_baseline(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
