"""Benchmark of the ragged paged-attention path on one MI355X.

Workload of ``value`` (one "step"): a continuous-batching decode step of the
Llama-3.2-1B attention geometry — 16 ragged sequences with lognormal context
lengths (median 2048, sigma 1, clipped to [32, 29600], seed 1), 32 query / 8
KV heads, head_dim 64, block_size 16, bf16, block tables drawn from a seeded
permutation of a pool twice the size needed.  For each of the 16 layers the
step appends one new K/V token per sequence and runs paged decode attention
over the grown sequences (one fused launch per layer).  16 layers give a
1.4 GB working set, far beyond the 256 MB last-level cache, so every step
reads its KV from HBM.

Prints one JSON line.  ``value`` = algorithmic bytes (decode K/V/Q/O/table
reads + append traffic) per second over the timed steps.  ``roofline`` is
for the decode-attention call, timed per launch with HIP events on its
stream.  Further fields: the same step as a captured serving step runs it
(``serving_plan_decode``), the 4-sequence decode call (``decode_small``),
the 16 x 29600 stress step on a pool of ~90% of free HBM, attention only and
through the whole model (``stress_16x29600``), the mixed chunked-prefill
step (``mixed_prefill_step``), longer prefills (``prefill_long``: 4 fresh
2048-token prompts, 4 chunks of 512 on 8192-token contexts), end-to-end
serving of the Llama-3.2-1B-shaped model (``e2e_llama1b_serving``) and the
reference algorithm's own times on the GPU and on the host cores
(``reference_path``, ``cpu_baseline``).
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
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE of the value leg's call, per rounding mode
TRAFFIC_PROFILES = {
    "reference": os.path.join("profiles", "decode_fused_kernel__decode_step_b16_lognormal__hbm_traffic.json"),
    "fast": os.path.join("profiles", "paged_decode_kernel__decode_step_b16_lognormal__hbm_traffic.json"),
}
# the kernels of one nie_paged_decode_append call, per rounding mode
DECODE_CALL_KERNELS = {
    "reference": "decode_fused_kernel (one launch: K phase, (max, sum) exchange between splits, P.V phase, last split sums)",
    "fast": "paged_decode_kernel + decode_merge_kernel",
}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=40)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=16)
    p.add_argument("--unfused-append", action="store_true",
                   help="decode step as nie_kv_append then nie_paged_decode (two launches per layer)")
    p.add_argument("--only", choices=["decode", "small", "stress", "mixed", "long", "e2e", "linear", "reference",
                                      "onepass"],
                   help="run one leg and print its JSON only")
    p.add_argument("--skip", action="append", default=[],
                   choices=["small", "stress", "stress-model", "mixed", "long", "e2e", "reference", "cpu", "lockstep"],
                   help="leave a leg out of the default line (repeatable)")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="target duration of the CPU baseline sample")
    p.add_argument("--pool-fraction", type=float, default=0.9,
                   help="stress step: KV pool as a fraction of the free device memory")
    p.add_argument("--stress-steps", type=int, default=256, help="stress step: decode steps (one append each)")
    p.add_argument("--lockstep-requests", type=int, default=16,
                   help="serving requests replayed on the reference algorithm (bf16 and fp32)")
    p.add_argument("--native-gemm", choices=["on", "off"], default="off",
                   help="serving legs: decode-step projections on nie_linear_rows (on) or torch's GEMM (off, the "
                        "reference's arithmetic)")
    p.add_argument("--rounding", choices=["reference", "fast"], default="reference",
                   help="bf16 attention probabilities: the reference's rounding point (normalised P cast to bf16, "
                        "two passes) or one pass with an online softmax")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run 4 device-to-device copies of MIB MiB (reference for HBM byte counters)")
    return p.parse_args()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def _median_us(pairs) -> float:
    import numpy as np

    return float(np.median([a.elapsed_time(b) for a, b in pairs])) * 1e3


# ---------------------------------------------------------------------------
# decode steps over a synthetic pool
# ---------------------------------------------------------------------------
class DecodeBench:
    """Device state for repeated append + decode steps over one workload.

    ``pool_blocks``: pool size (default: twice the blocks the steps need); the
    tables are a seeded permutation of the whole pool.  Only the blocks the
    tables use are filled with N(0, 1) values (the rest is never read), so a
    pool of most of HBM costs no fill time.
    """

    def __init__(self, wl, steps_total: int, device, seed: int, pool_blocks: int | None = None):
        import numpy as np
        import torch

        self.wl = wl
        self.device = device
        bs = wl.block_size
        rng = np.random.default_rng(seed + 500)
        need = [-(-(c + steps_total + 1) // bs) for c in wl.context_lens]
        self.num_blocks = pool_blocks or max(int(sum(need) * 2), wl.num_blocks)
        perm = rng.permutation(self.num_blocks)
        tables, cursor = [], 0
        for n in need:
            tables.append(perm[cursor : cursor + n])
            cursor += n
        width = max(len(t) for t in tables)
        table_arr = np.zeros((len(tables), width), dtype=np.int32)
        for r, t in enumerate(tables):
            table_arr[r, : len(t)] = t
        self.table_arr = table_arr
        shape = (wl.num_layers, self.num_blocks, bs, wl.kv_heads, wl.head_dim)
        gen = torch.Generator(device=device).manual_seed(seed)
        self.k_cache = torch.empty(shape, device=device, dtype=torch.bfloat16)
        self.v_cache = torch.empty(shape, device=device, dtype=torch.bfloat16)
        used = torch.from_numpy(np.unique(np.concatenate(tables)).astype(np.int64)).to(device)
        fill = (wl.num_layers, used.numel(), bs, wl.kv_heads, wl.head_dim)
        for cache in (self.k_cache, self.v_cache):
            cache[:, used] = torch.randn(fill, generator=gen, device=device, dtype=torch.bfloat16)
        self.tables = torch.from_numpy(table_arr).to(device)
        b = len(tables)
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

    def pool_bytes(self) -> int:
        return 2 * self.k_cache.numel() * self.k_cache.element_size()

    def prepared(self, s: int, serving_plan: bool = False, fused: bool = True):
        """The step's decode launch.  serving_plan: as a captured decode step of
        the serving path runs it (``generation.decode_graph``): sized for the
        512-rounded bound of the longest sequence, its work items read from
        the plan of the step's host lengths in device memory (written and
        copied here, before the step's launches); unfused, from the bound."""
        import numpy as np
        import torch

        from nano_infer_engine import _native
        from nano_infer_engine.paged_batch import decode_plan_bound

        if not serving_plan:
            return _native.PreparedDecode(self.k_cache, self.v_cache, self.tables, self.lens[s], self.max_len[s],
                                          self.total_len[s], self.wl.q_heads, self.scale,
                                          seq_lens_host=self.seq_lens_host[s])
        bound = decode_plan_bound(self.max_len[s])
        tables = self.tables
        width = -(-bound // self.wl.block_size)
        if tables.shape[1] < width:
            pad = torch.zeros((tables.shape[0], width - tables.shape[1]), dtype=tables.dtype, device=tables.device)
            tables = torch.cat([tables, pad], dim=1)
        plan = None
        if fused:
            host = np.zeros(_native.decode_plan_bytes() // 4, dtype=np.int32)
            _native.write_decode_plan(host.ctypes.data, host.nbytes, self.k_cache.dtype, self.wl.q_heads,
                                      self.wl.kv_heads, self.wl.head_dim, self.wl.block_size,
                                      np.asarray(self.seq_lens_host[s], dtype=np.int32), self.max_len[s],
                                      self.total_len[s])
            plan = torch.from_numpy(host.view(np.uint8)).to(self.k_cache.device)
        return _native.PreparedDecode(self.k_cache, self.v_cache, tables, self.lens[s], bound,
                                      bound * tables.shape[0], self.wl.q_heads, self.scale, device_plan=plan)

    def step(self, s: int, events: list | None = None, fused: bool = True, serving_plan: bool = False) -> None:
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
        decode = self.prepared(s, serving_plan, fused)
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


def _event_rate(bench, ev, first_step: int, steps: int, fused: bool):
    """(bytes per call, median call seconds, GB/s) of HIP-event-timed calls.

    The median: an event pair also spans the host's submission of the call,
    and a host stall (the garbage collector, a page fault) lengthens a few
    pairs to 100 us or more."""
    from nano_infer_engine import workloads

    avg = _median_us(ev) / 1e6
    per_call = sum(workloads.decode_bytes(bench.seq_lens_host[s]) for s in range(first_step, first_step + steps))
    per_call = per_call * bench.wl.num_layers / len(ev)
    if fused:
        per_call += workloads.append_bytes(len(bench.wl.context_lens))
    return per_call, avg, per_call / avg / 1e9


def _measured_traffic(rounding: str):
    """HBM bytes per decode call of the committed rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE)."""
    try:
        with open(os.path.join(REPO, TRAFFIC_PROFILES[rounding])) as f:
            data = json.load(f)
        return data.get("hbm_bytes_per_launch"), data.get("algorithmic_bytes_per_launch")
    except (OSError, ValueError):
        return None, None


def run_decode(args):
    """The ``value`` leg: configuration 2 over 16 layers, host-planned launches."""
    import torch

    from nano_infer_engine import _native, workloads

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    _native.load_library()
    wl = workloads.decode_ragged(num_layers=args.layers)
    # steps [0, W) warm up, [W, W+K) are the timed steps, [W+K, W+2K) are
    # timed again per call with HIP events and [W+2K, W+3K) with the serving
    # plan (kept out of the wall-clock pass, whose host and queue work the
    # events would add to)
    timed_end = args.warmup + args.steps
    total_steps = timed_end + 2 * args.steps
    bench = DecodeBench(wl, total_steps, device, seed=1)
    log(f"workload: {len(wl.context_lens)} seqs, contexts {wl.context_lens}, layers {args.layers}, "
        f"pool {bench.num_blocks} blocks ({bench.pool_bytes() / 1e9:.2f} GB)")
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
    for s in range(timed_end, timed_end + args.steps):
        bench.step(s, ev, fused=fused)
    torch.cuda.synchronize()
    bytes_per_call, avg_s, achieved = _event_rate(bench, ev, timed_end, args.steps, fused)

    serve_ev: list = []
    bench.step(timed_end + args.steps, fused=fused, serving_plan=True)  # warm the bound-planned launch
    for s in range(timed_end + args.steps, total_steps):
        bench.step(s, serve_ev, fused=fused, serving_plan=True)
    torch.cuda.synchronize()
    s_bytes, s_avg, s_gbs = _event_rate(bench, serve_ev, timed_end + args.steps, args.steps, fused)

    decode_bytes = sum(workloads.decode_bytes(bench.seq_lens_host[s]) for s in range(args.warmup, timed_end))
    decode_bytes *= args.layers
    append_bytes = workloads.append_bytes(len(wl.context_lens)) * args.layers * args.steps
    value = (decode_bytes + append_bytes) / elapsed / 1e9
    call = "nie_paged_decode_append" if fused else "nie_paged_decode"
    log(f"timed {args.steps} steps in {elapsed * 1e3:.2f} ms ({value:.0f} GB/s); {call} call avg "
        f"{avg_s * 1e6:.2f} us for {bytes_per_call / 1e6:.2f} MB -> {achieved:.0f} GB/s; serving plan "
        f"{s_avg * 1e6:.2f} us -> {s_gbs:.0f} GB/s")
    traffic, traffic_alg = _measured_traffic(args.rounding)
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
            "kernel": f"{call} call: {DECODE_CALL_KERNELS[args.rounding]} (HIP events around the call)",
            "rounding": args.rounding,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": f"{TRAFFIC_PROFILES[args.rounding]}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this call on this "
                              f"workload (algorithmic bytes there: {traffic_alg}), scaled by a 1 GiB copy",
            "algorithmic_bytes_per_launch": int(bytes_per_call),
            "avg_launch_us": round(avg_s * 1e6, 3),
        },
        "serving_plan_decode": {
            "plan": "as a captured serving decode step runs it: launch sized for the 512-rounded bound, work "
                    "items from the step's host plan in device memory",
            "avg_launch_us": round(s_avg * 1e6, 3), "achieved_GBs": round(s_gbs, 1),
            "frac": round(s_gbs / HBM_PEAK_GBS, 4),
        },
    }
    del bench
    torch.cuda.empty_cache()
    return result


def run_decode_small(args):
    """Configuration 1: 4 sequences {17, 64, 129, 500}, 256-block pool, one call, bf16."""
    import torch

    from nano_infer_engine import _native, workloads

    device = torch.device("cuda:0")
    wl = workloads.decode_small()
    kc, vc = wl.pool(torch.bfloat16, device)
    q, _, _ = wl.new_tokens(torch.bfloat16, device)
    tables = torch.from_numpy(wl.table_array()).to(device)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=device)
    decode = _native.PreparedDecode(kc, vc, tables, lens, max(wl.seq_lens), sum(wl.seq_lens), wl.q_heads,
                                    wl.head_dim**-0.5, seq_lens_host=wl.seq_lens)
    out = torch.empty_like(q)
    for _ in range(10):
        decode(q, 0, out)
    ev = []
    for _ in range(100):
        e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        e[0].record()
        decode(q, 0, out)
        e[1].record()
        ev.append(e)
    torch.cuda.synchronize()
    us = _median_us(ev)
    nbytes = workloads.decode_bytes(wl.seq_lens)
    log(f"decode small: {us:.2f} us for {nbytes / 1e6:.3f} MB")
    return {"avg_launch_us": round(us, 2), "bytes_per_launch": nbytes,
            "achieved_GBs": round(nbytes / us / 1e3, 1), "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}


# ---------------------------------------------------------------------------
# configuration 5: 16 x 29600 contexts on a pool of most of HBM
# ---------------------------------------------------------------------------
def _free_bytes() -> int:
    import torch

    torch.cuda.empty_cache()
    return torch.cuda.mem_get_info()[0]


def run_stress(args):
    """Decode over 16 x 29600-token contexts (970 MB per layer-step) with one
    append per step, on one layer whose pool is ``--pool-fraction`` of the
    free device memory with fully permuted tables."""
    import torch

    from nano_infer_engine import workloads

    device = torch.device("cuda:0")
    steps, warmup = args.stress_steps, 5
    wl = workloads.decode_long(num_layers=1)
    block_bytes = 2 * wl.block_size * wl.kv_heads * wl.head_dim * 2  # K + V of one block, bf16
    bench = None
    for fraction in (args.pool_fraction, 0.8 * args.pool_fraction, 0.6 * args.pool_fraction):
        pool_blocks = int(_free_bytes() * fraction) // block_bytes
        try:
            bench = DecodeBench(wl, steps + warmup, device, seed=4, pool_blocks=pool_blocks)
            break
        except torch.OutOfMemoryError:
            log(f"stress pool of {fraction:.0%} of free memory did not fit; trying less")
            torch.cuda.empty_cache()
    if bench is None:
        raise RuntimeError("no stress pool fits")
    args = argparse.Namespace(**{**vars(args), "pool_fraction": fraction})
    log(f"stress pool: {pool_blocks} blocks = {bench.pool_bytes() / 1e9:.1f} GB "
        f"({args.pool_fraction:.0%} of free), tables over the whole pool")
    fused = not args.unfused_append
    for s in range(warmup):
        bench.step(s, fused=fused)
    torch.cuda.synchronize()
    ev: list = []
    for s in range(warmup, warmup + steps):
        bench.step(s, ev, fused=fused)
    torch.cuda.synchronize()
    per_call, avg, gbs = _event_rate(bench, ev, warmup, steps, fused)
    log(f"stress 16x29600: {avg * 1e6:.1f} us per layer-step over {steps} steps, {gbs:.0f} GB/s")
    out = {"avg_launch_us": round(avg * 1e6, 2), "bytes_per_launch": int(per_call),
           "achieved_GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "steps": steps,
           "pool_blocks": pool_blocks, "pool_GB": round(bench.pool_bytes() / 1e9, 1),
           "pool_fraction_of_free": args.pool_fraction}
    del bench
    torch.cuda.empty_cache()
    return out


def run_stress_model(args):
    """The 16 x 29600 decode through the whole Llama-3.2-1B-shaped model:
    captured decode steps (``DecodeGraphRunner``) over a 16-layer cache of
    ``--pool-fraction`` of the free memory whose allocator hands out blocks in
    a seeded random order; the contexts' K/V are N(0, 1) values."""
    import numpy as np
    import torch

    from nano_infer_engine import workloads
    from nano_infer_engine.generation.decode_graph import DecodeGraphRunner
    from nano_infer_engine.paged_cache import PagedKVCache

    device = torch.device("cuda:0")
    model = workloads.serving_model(device)
    cfg = model.config
    steps, ctx = args.stress_steps, 29600
    block_bytes = 2 * cfg.num_layers * 16 * cfg.kv_head_num * cfg.head_dim * 2
    # leave room for activations and a few captured graphs
    pool_blocks = int((_free_bytes() - (4 << 30)) * args.pool_fraction) // block_bytes
    cache = PagedKVCache(pool_blocks, 16, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, torch.bfloat16, device)
    # a permuted free list: take every block, give them back in random order
    everything = cache.allocator.allocate(pool_blocks)
    cache.allocator.free(np.random.default_rng(5).permutation(everything).tolist())
    ids = tuple(f"long-{i}" for i in range(16))
    for sid in ids:
        cache.ensure_capacity(sid, ctx + steps + 1)
        cache.advance(sid, ctx)
    used = torch.tensor(sorted(b for sid in ids for b in cache.get_block_table(sid)), device=device)
    gen = torch.Generator(device=device).manual_seed(4)
    for layer in range(cfg.num_layers):
        for pool in (cache.keys, cache.values):
            pool[layer, used] = torch.randn((used.numel(), 16, cfg.kv_head_num, cfg.head_dim), generator=gen,
                                            device=device, dtype=torch.bfloat16)
    runner = DecodeGraphRunner(model, cache, 16)
    tokens = torch.randint(0, cfg.vocab_size, (16,), generator=gen, device=device)
    times = []
    for s in range(steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _, tokens = runner.step(tokens, ids)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times[3:])) * 1e3
    kv = workloads.decode_bytes([ctx + steps // 2] * 16) * cfg.num_layers
    log(f"stress full model: {ms:.3f} ms per decode step (median of {steps - 3}; {runner.captures} captures), "
        f"pool {pool_blocks} blocks = {2 * cache.keys.numel() * 2 / 1e9:.1f} GB")
    out = {"ms_per_step": round(ms, 3), "output_tok_per_s": round(16 / ms * 1e3, 1), "steps": steps,
           "attention_bytes_per_step": kv, "pool_blocks": pool_blocks,
           "pool_GB": round(2 * cache.keys.numel() * 2 / 1e9, 1), "graph_captures": runner.captures}
    del runner, cache, model
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# configuration 3: mixed chunked-prefill step
# ---------------------------------------------------------------------------
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
    p_us, d_us = _median_us(pev), _median_us(dev_)
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


def run_prefill_long(args):
    """The varlen prefill call on longer prefills than the mixed step's, where
    the per-call fixed costs (prologue, split partials, merge) weigh less:
    4 fresh 2048-token prompts, and 4 chunks of 512 tokens on 8192-token
    contexts; bf16, one layer, launches planned from host lengths."""
    import numpy as np
    import torch

    from nano_infer_engine import _native, workloads

    device = torch.device("cuda:0")
    out = {}
    for name, wl in (("prompts_4x2048", workloads.prefill_prompts()),
                     ("chunks_4x512_on_8192", workloads.prefill_long_context())):
        kc, vc = wl.pool(torch.bfloat16, device)
        q, k_new, v_new = wl.new_tokens(torch.bfloat16, device)
        _native.kv_append(kc, vc, 0, k_new, v_new, torch.from_numpy(wl.slots()).to(device))
        cu_host = [0] + np.cumsum(wl.query_lens).tolist()
        cu = torch.tensor(cu_host, dtype=torch.int64, device=device)
        ctx = torch.tensor(wl.context_lens, dtype=torch.int32, device=device)
        tables = torch.from_numpy(wl.table_array()).to(device)
        prefill = _native.PreparedPrefill(kc, vc, cu, ctx, tables, wl.num_tokens, max(wl.query_lens),
                                          max(wl.seq_lens), wl.q_heads, wl.head_dim**-0.5,
                                          cu_seqlens_host=cu_host, context_lens_host=wl.context_lens)
        o = torch.empty_like(q)
        for _ in range(5):
            prefill(q, 0, o)
        ev = []
        for _ in range(30):
            e = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            e[0].record()
            prefill(q, 0, o)
            e[1].record()
            ev.append(e)
        torch.cuda.synchronize()
        us = _median_us(ev)
        flops = workloads.prefill_flops(wl.context_lens, wl.query_lens)
        tflops = flops / (us * 1e-6) / 1e12
        log(f"prefill {name}: {us:.1f} us = {tflops:.1f} TFLOP/s ({flops / 1e9:.2f} GFLOP)")
        out[name] = {"avg_launch_us": round(us, 2), "flops_per_launch": flops, "achieved_TFLOPs": round(tflops, 2),
                     "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
        del kc, vc, prefill
        torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# configuration 4: end-to-end serving
# ---------------------------------------------------------------------------
def serve(model, prompts, device, max_new_tokens, graphs=True):
    """Serve every prompt through the continuous-batching scheduler; returns (seconds, steps, requests).

    With ``graphs`` the all-decode steps replay captured HIP graphs (captures
    happen inside the timed region, as in a fresh server)."""
    import torch

    from nano_infer_engine import workloads
    from nano_infer_engine.generation import ContinuousBatchingScheduler, GenerationConfig
    from nano_infer_engine.paged_cache import PagedKVCache

    cfg = model.config
    cache = PagedKVCache(workloads.serving_cache_blocks(prompts, max_new_tokens), 16, cfg.num_layers,
                         cfg.kv_head_num, cfg.head_dim, torch.bfloat16, device)
    gen = GenerationConfig(max_new_tokens=max_new_tokens, eos_token_id=None,
                           prefill_chunk_size=workloads.SERVING_CHUNK,
                           max_prefill_tokens_per_step=workloads.SERVING_STEP_BUDGET)
    sched = ContinuousBatchingScheduler(model, gen, cache, max_batch_size=workloads.SERVING_MAX_BATCH,
                                        decode_graphs=graphs)
    reqs = [sched.add_request(f"request-{i}", p) for i, p in enumerate(prompts)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    steps = 0
    while sched.has_work:
        sched.step()
        steps += 1
    torch.cuda.synchronize()
    return time.perf_counter() - t0, steps, reqs


def run_e2e(args):
    """Configuration 4: 64 requests x 256 greedy tokens, graph-replayed and eager decode steps."""
    import torch

    import nano_infer_engine.layers.linear as linear_module
    from nano_infer_engine import workloads

    linear_module.USE_NATIVE = args.native_gemm == "on"
    device = torch.device("cuda:0")
    model = workloads.serving_model(device)
    prompts = workloads.serving_prompts(device, model.config.vocab_size)
    serve(model, prompts[:2], device, 8)  # warm-up: library load, GEMM heuristics
    secs, steps, reqs = serve(model, prompts, device, workloads.SERVING_NEW_TOKENS)
    out_tokens = sum(r.generated_tokens for r in reqs)
    tok_s = out_tokens / secs
    log(f"e2e: {out_tokens} output tokens from {len(prompts)} requests in {secs:.2f} s "
        f"({steps} steps) -> {tok_s:.0f} tok/s")
    eager_secs, _, eager_reqs = serve(model, prompts, device, workloads.SERVING_NEW_TOKENS, graphs=False)
    eager_tok_s = sum(r.generated_tokens for r in eager_reqs) / eager_secs
    same_modes = all(torch.equal(a.sequence, b.sequence) for a, b in zip(reqs, eager_reqs))
    log(f"e2e eager (no decode graphs): {eager_secs:.2f} s -> {eager_tok_s:.0f} tok/s; "
        f"tokens identical to the graph run: {same_modes}")
    del model
    torch.cuda.empty_cache()
    return {
        "output_tok_per_s": round(tok_s, 1),
        "output_tok_per_s_eager": round(eager_tok_s, 1),
        "eager_tokens_identical": same_modes,
        "output_tokens": out_tokens,
        "seconds": round(secs, 3),
        "scheduler_steps": steps,
        "decode_gemm": "nie_linear_rows" if linear_module.USE_NATIVE else "torch",
        "workload": "Llama-3.2-1B shape, bf16, random N(0, 0.02) weights; 64 requests, prompts U[128, 2048] "
                    "(seed 3), 256 greedy tokens each, max batch 16, prefill chunk 128, 512 prefill tokens/step",
    }


# ---------------------------------------------------------------------------
# the reference algorithm's own times (the oracle, on the GPU and the host)
# ---------------------------------------------------------------------------
def _cpu_model() -> str:
    """The host CPU's model name with its family / model / stepping numbers
    (a virtualised host may report only a generic name)."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" in line:
                    key, value = (s.strip() for s in line.split(":", 1))
                    fields.setdefault(key, value)
                if not line.strip() and fields:
                    break
    except OSError:
        return "unknown"
    name = fields.get("model name", "unknown")
    ids = [f"{k.split()[-1]} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    return f"{name} ({', '.join(ids)})" if ids else name


def _time_host(fn, min_seconds: float, max_reps: int = 1000, warmup: bool = True):
    """(seconds per call, calls) of fn on the host, after one warm-up call."""
    if warmup:
        fn()
    done, t0 = 0, time.perf_counter()
    while done < max_reps:
        fn()
        done += 1
        if time.perf_counter() - t0 >= min_seconds:
            break
    return (time.perf_counter() - t0) / done, done


def _time_gpu(fn, min_seconds: float, max_reps: int = 100):
    import torch

    def synced():
        fn()
        torch.cuda.synchronize()

    return _time_host(synced, min_seconds, max_reps)


def run_cpu_baseline(args):
    """The oracle (the reference's per-block decode loop, torch bf16 on the
    host cores) on a bounded sample of the ``value`` workload."""
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
    per_call, done = _time_host(lambda: reference_ops.batched_paged_attention_reference(q, kc, vc, tables, lens, 0),
                                args.cpu_seconds)
    gbs = workloads.decode_bytes(lens) / per_call / 1e9
    cpu = _cpu_model()
    log(f"cpu baseline: {done} layer-steps, {per_call * 1e3:.1f} ms each on {threads} threads ({cpu}) "
        f"-> {gbs:.3f} GB/s")
    return {
        "value": round(gbs, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": cpu,
        "sample": f"{done} single-layer decode attention calls over the same 16 sequences "
                  f"({sum(lens)} tokens), the reference's per-block loop in torch bf16 on the host, "
                  f"{done * per_call:.1f} s",
    }


def run_reference_path(args):
    """The reference algorithm (the oracle's restatement, torch) timed on the
    GPU and on the host cores for configurations 1, 2, 3 and 5 (one layer;
    configuration 5 one step), beside this build's HIP figures."""
    import torch

    from nano_infer_engine import workloads
    from oracle import reference_ops

    device = torch.device("cuda:0")
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    out = {"cpu_model": _cpu_model(), "cpu_threads": threads}

    def decode_case(name, wl, cpu_seconds, gpu_seconds, host_warmup=True):
        # N(0, 1) pool and queries drawn on the device (a 16 x 29600 pool
        # is 1.9 GB) and copied to the host for the CPU leg
        gen = torch.Generator(device=device).manual_seed(wl.seed)
        shape = (1, wl.num_blocks, wl.block_size, wl.kv_heads, wl.head_dim)
        gk, gv = (torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16) for _ in range(2))
        gq = torch.randn((len(wl.seq_lens), wl.q_heads, wl.head_dim), generator=gen, device=device,
                         dtype=torch.bfloat16)
        kc, vc, q = gk.cpu(), gv.cpu(), gq.cpu()
        tables, lens = tuple(tuple(t) for t in wl.tables), tuple(wl.seq_lens)
        g_s, g_n = _time_gpu(lambda: reference_ops.batched_paged_attention_reference_matmul(gq, gk, gv, tables, lens,
                                                                                          0), gpu_seconds)
        c_s, c_n = _time_host(lambda: reference_ops.batched_paged_attention_reference(q, kc, vc, tables, lens, 0),
                              cpu_seconds, max_reps=50, warmup=host_warmup)
        nbytes = workloads.decode_bytes(lens)
        log(f"reference {name}: GPU torch {g_s * 1e3:.2f} ms ({g_n} calls), CPU {c_s * 1e3:.1f} ms ({c_n} calls)")
        out[name] = {"bytes_per_call": nbytes, "gpu_torch_ms": round(g_s * 1e3, 3),
                     "gpu_torch_GBs": round(nbytes / g_s / 1e9, 2), "cpu_ms": round(c_s * 1e3, 2),
                     "cpu_GBs": round(nbytes / c_s / 1e9, 4)}
        del gk, gv
        torch.cuda.empty_cache()

    decode_case("config1_decode_small", workloads.decode_small(), 2.0, 1.0)
    decode_case("config2_decode_step", workloads.decode_ragged(), 2.0, 2.0)
    decode_case("config5_decode_16x29600", workloads.decode_long(), 1.0, 2.0, host_warmup=False)

    wl = workloads.mixed_prefill()
    kc, vc = wl.pool(torch.bfloat16)
    q, k_new, v_new = wl.new_tokens(torch.bfloat16)
    args_cpu = (q, k_new, v_new, kc, vc)
    args_gpu = tuple(t.to(device) for t in args_cpu)
    meta = (0, wl.tables, wl.context_lens, wl.query_lens, wl.head_dim**-0.5)
    g_s, _ = _time_gpu(lambda: reference_ops.ragged_attention_reference_vectorized(*args_gpu, *meta), 2.0)
    c_s, _ = _time_host(lambda: reference_ops.ragged_attention_reference(*args_cpu, *meta), 2.0, max_reps=20)
    flops = workloads.prefill_flops(wl.context_lens[:4], wl.query_lens[:4])
    log(f"reference config3: GPU torch {g_s * 1e3:.2f} ms, CPU {c_s * 1e3:.1f} ms")
    out["config3_mixed_step"] = {"gpu_torch_ms": round(g_s * 1e3, 3), "cpu_ms": round(c_s * 1e3, 2),
                                 "prefill_flops": flops, "note": "whole step (4 prefill chunks + 12 decode rows); "
                                 "the GPU leg gathers with one index_select per request, the host leg token by token "
                                 "as the reference does"}
    del args_gpu
    torch.cuda.empty_cache()
    return out


def run_lockstep(args):
    """Configuration 4's numerics and the reference path's end-to-end rate:
    ``--lockstep-requests`` requests served by the product, every step
    replayed on the reference algorithm in bf16 and in fp32."""
    import torch

    import nano_infer_engine.layers.linear as linear_module
    from nano_infer_engine import workloads
    from nano_infer_engine.paged_cache import PagedKVCache
    from oracle import lockstep

    linear_module.USE_NATIVE = args.native_gemm == "on"
    device = torch.device("cuda:0")
    model = workloads.serving_model(device)
    cfg = model.config
    prompts = workloads.serving_prompts(device, cfg.vocab_size, count=args.lockstep_requests)
    blocks = workloads.serving_cache_blocks(prompts, workloads.SERVING_NEW_TOKENS)

    def cache(dtype):
        return PagedKVCache(blocks, 16, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, dtype, device)

    serve(model, prompts[:2], device, 8)  # warm-up
    secs, _, reqs = serve(model, prompts, device, workloads.SERVING_NEW_TOKENS)
    ours = sum(r.generated_tokens for r in reqs) / secs
    report = lockstep.run_lockstep(model, prompts, cache, max_new_tokens=workloads.SERVING_NEW_TOKENS,
                                   max_batch_size=workloads.SERVING_MAX_BATCH, chunk=workloads.SERVING_CHUNK,
                                   budget=workloads.SERVING_STEP_BUDGET, variant=True)
    summary = report.summary()
    tokens = summary["sampled_rows"]
    ref_rate = tokens / report.reference_seconds
    log(f"lockstep: {summary['requests']} requests, top-1 agreement product/reference "
        f"{summary['top1_agreement_product_reference']:.4f}, product/truth {summary['top1_agreement_product_truth']:.4f}, "
        f"reference/truth {summary['top1_agreement_reference_truth']:.4f}; reference path {ref_rate:.0f} tok/s "
        f"against {ours:.0f} tok/s")
    firsts = summary.pop("first_divergence")
    summary["first_divergence_tokens"] = sorted(v["token"] for v in firsts.values() if v)
    summary["reference_output_tok_per_s"] = round(ref_rate, 1)
    summary["product_output_tok_per_s"] = round(ours, 1)
    summary["speedup"] = round(ours / ref_rate, 2)
    summary["decode_gemm"] = "nie_linear_rows" if linear_module.USE_NATIVE else "torch"
    summary["method"] = ("the product serves the requests as shipped; each step is replayed, teacher-forced, on "
                         "the reference algorithm (bf16; one index_select per request instead of the per-token "
                         "gather) and in fp32 (the truth); the reference rate is the sum of its forwards' times")
    del model
    torch.cuda.empty_cache()
    return summary


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
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "torch_us": round(res["torch"], 2)}
        log(f"{name:15s} {n}x{k}: nie_linear_rows {res['nie_linear_rows']:.2f} us ({gbs:.0f} GB/s), "
            f"torch {res['torch']:.2f} us")
        del ws
        torch.cuda.empty_cache()
    return out


def run_one_pass_rounding(args):
    """The cost of the reference's rounding point: configurations 2, 3 and 5
    (and the long prefills) again with the one-pass rounding (online softmax,
    NIE_ROUND_FAST), the kernels the reference rounding replaced."""
    from nano_infer_engine import _native

    _native.set_attention_rounding("fast")
    try:
        fast = argparse.Namespace(**{**vars(args), "rounding": "fast"})
        d = run_decode(fast)
        s = run_stress(fast)
        m = run_mixed(fast)
        lp = run_prefill_long(fast)
    finally:
        _native.set_attention_rounding(args.rounding)
    return {
        "rounding": "fast (one pass, online softmax)",
        "config2_decode_call": {"avg_launch_us": d["roofline"]["avg_launch_us"], "frac": d["roofline"]["frac"],
                                "step_GBs": d["value"]},
        "config2_serving_plan_call": {"avg_launch_us": d["serving_plan_decode"]["avg_launch_us"],
                                      "frac": d["serving_plan_decode"]["frac"]},
        "config5_16x29600_call": {"avg_launch_us": s["avg_launch_us"], "frac": s["frac"]},
        "config3_prefill_call": {"avg_launch_us": m["prefill"]["avg_launch_us"], "frac": m["prefill"]["frac"]},
        "config3_decode_rows_call": {"avg_launch_us": m["decode_rows"]["avg_launch_us"],
                                     "frac": m["decode_rows"]["frac"]},
        "prefill_prompts_4x2048": {"avg_launch_us": lp["prompts_4x2048"]["avg_launch_us"],
                                   "frac": lp["prompts_4x2048"]["frac"]},
        "prefill_chunks_4x512_on_8192": {"avg_launch_us": lp["chunks_4x512_on_8192"]["avg_launch_us"],
                                         "frac": lp["chunks_4x512_on_8192"]["frac"]},
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
    from nano_infer_engine import _native

    _native.load_library()
    _native.set_attention_rounding(args.rounding)
    only = {
        "decode": ("decode", run_decode), "small": ("decode_small", run_decode_small),
        "stress": ("stress_16x29600", lambda a: {"attention": run_stress(a), "full_model": run_stress_model(a)}),
        "mixed": ("mixed_prefill_step", run_mixed), "long": ("prefill_long", run_prefill_long),
        "e2e": ("e2e_llama1b_serving", run_e2e),
        "linear": ("decode_projections", run_linear),
        "reference": ("reference_path", lambda a: {**run_reference_path(a), "serving_lockstep": run_lockstep(a)}),
        "onepass": ("one_pass_rounding", run_one_pass_rounding),
    }
    if args.only:
        key, fn = only[args.only]
        print(json.dumps({key: fn(args)}), flush=True)
        return
    skip = set(args.skip)
    result = run_decode(args)
    if "small" not in skip:
        result["decode_small"] = run_decode_small(args)
    if "stress" not in skip:
        result["stress_16x29600"] = run_stress(args)
        if "stress-model" not in skip:
            result["stress_16x29600"]["full_model"] = run_stress_model(args)
    if "mixed" not in skip:
        result["mixed_prefill_step"] = run_mixed(args)
    if "long" not in skip:
        result["prefill_long"] = run_prefill_long(args)
    if "e2e" not in skip:
        result["e2e_llama1b_serving"] = run_e2e(args)
    if "reference" not in skip:
        result["reference_path"] = run_reference_path(args)
        if "lockstep" not in skip:
            result["reference_path"]["serving_lockstep"] = run_lockstep(args)
    if "onepass" not in skip and args.rounding == "reference":
        result["one_pass_rounding"] = run_one_pass_rounding(args)
    result["cpu_baseline"] = None if "cpu" in skip else run_cpu_baseline(args)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
