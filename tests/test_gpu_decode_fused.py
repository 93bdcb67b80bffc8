"""The one-launch reference-rounding decode (decode_fused_kernel) against the
two launches it replaces (scores pass, P.V pass) and against the oracle,
through the C ABI.

Bars: outputs and cache writes bit-identical to the pass launches (the same
arithmetic in the same order); outputs within the bf16 bar (2e-2 max-abs) of
the reference-algorithm oracle; the workspace's control region left zero by
every call.  The shapes the one-launch kernel is not built for (GQA groups
above 4, head_dim 128, block sizes that split a 16-key tile) must take the
pass launches.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_infer_engine import _native, workloads
from oracle import reference_ops

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _log(msg: str) -> None:
    print(msg, flush=True)


@pytest.fixture(autouse=True)
def _reference_rounding():
    """Every test here runs with the reference rounding and the default switches."""
    before = _native.attention_rounding()
    _native.set_attention_rounding("reference")
    _native.set_decode_fused(True)
    _native.set_decode_fused_spin(32768)
    yield
    _native.set_decode_fused(True)
    _native.set_decode_fused_spin(32768)
    _native.set_attention_rounding(before)


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    ints = {torch.bfloat16: torch.int16, torch.float32: torch.int32}[a.dtype]
    return a.dtype == b.dtype and torch.equal(a.cpu().view(ints), b.cpu().view(ints))


def _decode_oracle(wl, kc_cpu, vc_cpu, q_cpu):
    return reference_ops.batched_paged_attention_reference(
        q_cpu, kc_cpu, vc_cpu, tuple(tuple(t) for t in wl.tables), tuple(wl.seq_lens), 0
    )


def _control_regions_zero() -> bool:
    """Every cached workspace's counters are zero (the region's last 128-byte
    line holds only the count of waits that gave up)."""
    ctl = _native.workspace_control_bytes()
    return all(int(ws[: ctl - 128].count_nonzero().item()) == 0 for ws in _native._decode_workspaces.values())


def _gave_up_counts() -> list[int]:
    ctl = _native.workspace_control_bytes()
    return [int(ws[ctl - 128 : ctl - 124].view(torch.int32).item()) for ws in _native._decode_workspaces.values()]


def _fused_and_passes(fn):
    """fn() with the one-launch decode on, then off: both results and the paths taken."""
    fused = fn()
    torch.cuda.synchronize()
    fused_path = _native.decode_last_path()
    _native.set_decode_fused(False)
    try:
        passes = fn()
        torch.cuda.synchronize()
        passes_path = _native.decode_last_path()
    finally:
        _native.set_decode_fused(True)
    return fused, passes, fused_path, passes_path


def _workload(base: str):
    if base == "lognormal":  # the 16-sequence continuous-batching step, 43k tokens
        return workloads.decode_ragged(seed=7)
    if base == "small":
        return workloads.decode_small()
    if base == "long":
        return workloads.ragged([9000, 5000, 31, 16, 2500, 700], [1] * 6, seed=21, pool_factor=1.3)
    if base == "bs32":
        return workloads.ragged([3000, 33, 1024], [1] * 3, seed=25, pool_factor=1.5, block_size=32)
    if base == "group2":
        return workloads.ragged([1500, 40, 777], [1] * 3, seed=27, pool_factor=1.5, q_heads=8, kv_heads=4)
    if base == "many_short":  # 100 rows, most of them one split
        rng = np.random.default_rng(26)
        return workloads.ragged([int(x) for x in rng.integers(0, 300, 100)], [1] * 100, seed=26, pool_factor=1.3)
    if base == "few_long":  # one sequence of 39 splits at the smallest split length, in a small call
        return workloads.ragged([2490, 20, 100], [1] * 3, seed=28, pool_factor=1.3)
    if base == "gqa16":
        return workloads.ragged([1500, 40, 777], [1] * 3, seed=22, pool_factor=1.5, q_heads=16, kv_heads=1)
    if base == "d128":
        return workloads.ragged([2000, 15, 640], [1] * 3, seed=23, pool_factor=1.5, q_heads=8, kv_heads=8,
                                head_dim=128)
    if base == "bs8":
        return workloads.ragged([1200, 3, 400], [1] * 3, seed=24, pool_factor=1.5, block_size=8)
    raise ValueError(base)


FUSED_CASES = ["lognormal", "lognormal_host", "small", "small_host", "long_host", "bs32", "group2", "many_short"]
PASS_CASES = ["gqa16", "d128", "bs8"]


def _run_case(case: str, append: str):
    host_plan = case.endswith("_host")
    wl = _workload(case[: -len("_host")] if host_plan else case)
    dtype = torch.bfloat16
    kc, vc = wl.pool(dtype)
    q, k_new, v_new = wl.new_tokens(dtype)
    tables = torch.from_numpy(wl.table_array()).to(DEV)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)
    host = list(wl.seq_lens) if host_plan else None
    rope_tables = None
    if append == "rope":
        from nano_infer_engine.layers.rope import RopeScale

        rope_tables = RopeScale(wl.head_dim).tables(DEV, dtype, max(wl.seq_lens))
    dq = q.to(DEV)

    def run():
        k, v = kc.to(DEV), vc.to(DEV)
        kw = {}
        if append != "none":
            kw = dict(new_kv=(k_new.to(DEV), v_new.to(DEV)), rope_tables=rope_tables)
        out = _native.paged_decode(dq, k, v, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens),
                                   wl.head_dim**-0.5, seq_lens_host=host, **kw)
        return out, k, v

    return wl, kc, vc, q, run


@pytest.mark.parametrize("case", FUSED_CASES)
@pytest.mark.parametrize("append", ["none", "append", "rope"])
def test_fused_decode_matches_pass_launches(case, append):
    """One launch == the scores and P.V launches, bit for bit (outputs and
    cache writes), within the bf16 bar of the oracle, control region zero."""
    _log(f"fused decode vs passes: {case} {append}")
    wl, kc, vc, q, run = _run_case(case, append)
    (o1, k1, v1), (o2, k2, v2), p1, p2 = _fused_and_passes(run)
    _log(f"  paths: {p1} / {p2}")
    assert p1 == "fused" and p2 == "passes"
    assert _same_bits(o1, o2), "one-launch output differs from the pass launches"
    assert _same_bits(k1, k2) and _same_bits(v1, v2), "one-launch cache writes differ from the pass launches"
    assert _control_regions_zero()
    if append == "none":
        err = (o1.cpu().float() - _decode_oracle(wl, kc, vc, q).float()).abs().max().item()
        _log(f"  max_abs_err={err:.3e}")
        assert err <= 2e-2


@pytest.mark.parametrize("case", PASS_CASES)
def test_shapes_outside_the_fused_kernel_take_the_passes(case):
    _log(f"fused decode ineligible: {case}")
    wl, kc, vc, q, run = _run_case(case, "none")
    out, _, _ = run()
    torch.cuda.synchronize()
    assert _native.decode_last_path() == "passes"
    err = (out.cpu().float() - _decode_oracle(wl, kc, vc, q).float()).abs().max().item()
    assert err <= 2e-2


@pytest.mark.parametrize("case", ["lognormal", "long_host", "many_short"])
@pytest.mark.parametrize("append", ["none", "rope"])
def test_fused_decode_waits_that_give_up(case, append):
    """With a poll limit of 0 every split that waits for others gives up at
    once and forms their (max, sum) pairs itself from K: the outputs stay
    bit-identical to the pass launches', and the give-up count grows."""
    _log(f"fused decode, waits give up: {case} {append}")
    wl, kc, vc, q, run = _run_case(case, append)
    run()  # creates the cached workspace
    torch.cuda.synchronize()
    before = sum(_gave_up_counts())
    _native.set_decode_fused_spin(0)
    try:
        (o1, k1, v1), (o2, k2, v2), p1, p2 = _fused_and_passes(run)
    finally:
        _native.set_decode_fused_spin(32768)
    after = sum(_gave_up_counts())
    _log(f"  paths: {p1} / {p2}, waits given up: {after - before}")
    assert p1 == "fused" and p2 == "passes"
    assert after > before
    assert _same_bits(o1, o2)
    assert _same_bits(k1, k2) and _same_bits(v1, v2)
    assert _control_regions_zero()


def test_fused_decode_back_to_back_calls():
    """Many one-launch calls on one stream with no host synchronisation (the
    counters one call's sum kernel clears are the next call's starting
    state), alternating long and short batches: every output equals its
    single-call result bit for bit, and the control regions end zero."""
    _log("fused decode back to back")
    cases = [workloads.decode_ragged(seed=s) for s in (2, 4)] + [workloads.decode_small()]
    prepared = []
    for wl in cases:
        kc, vc = wl.pool(torch.bfloat16)
        q, _, _ = wl.new_tokens(torch.bfloat16)
        prepared.append((wl, kc.to(DEV), vc.to(DEV), q.to(DEV), torch.from_numpy(wl.table_array()).to(DEV),
                         torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)))

    def call(p, host):
        wl, dk, dv, dq, tables, lens = p
        return _native.paged_decode(dq, dk, dv, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens),
                                    wl.head_dim**-0.5, seq_lens_host=list(wl.seq_lens) if host else None)

    for host in (True, False):
        single = []
        for p in prepared:
            single.append(call(p, host))
            torch.cuda.synchronize()
            assert _native.decode_last_path() == "fused"
        outs = [call(prepared[i % len(prepared)], host) for i in range(24)]
        torch.cuda.synchronize()
        for i, got in enumerate(outs):
            assert _same_bits(got, single[i % len(prepared)]), i
        assert _control_regions_zero()


# --- the one-pass rounding: split partials merged by the last split -------

# small calls take the merge by the last split by default; the others only
# with the switch at 2 (forced), which these tests use to run the merge over
# many splits (several batches of 32 at head_dim 64)
MERGED_SMALL = ["small_host"]
MERGED_FORCED = ["small", "few_long", "few_long_host", "lognormal", "lognormal_host", "long_host", "many_short", "group2", "gqa16", "d128", "bs8", "bs32"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("case", MERGED_SMALL + MERGED_FORCED)
@pytest.mark.parametrize("append", ["none", "rope"])
def test_one_pass_merge_by_last_split_matches_merge_launch(case, append, dtype):
    """One-pass decode (fp32, and bf16 with the one-pass rounding): the
    merge of split partials by the split that finishes last, inside the
    decode kernel, equals the merge launch bit for bit (outputs and cache
    writes), within the oracle's bar, control regions zero."""
    _log(f"one-pass merged by the last split: {case} {append} {dtype}")
    _native.set_attention_rounding("fast")
    if case in MERGED_FORCED:
        _native.set_decode_fused(2)
    host_plan = case.endswith("_host")
    wl = _workload(case[: -len("_host")] if host_plan else case)
    kc, vc = wl.pool(dtype)
    q, k_new, v_new = wl.new_tokens(dtype)
    tables = torch.from_numpy(wl.table_array()).to(DEV)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)
    host = list(wl.seq_lens) if host_plan else None
    rope_tables = None
    if append == "rope":
        from nano_infer_engine.layers.rope import RopeScale

        rope_tables = RopeScale(wl.head_dim).tables(DEV, dtype, max(wl.seq_lens))
    dq = q.to(DEV)

    def run():
        k, v = kc.to(DEV), vc.to(DEV)
        kw = {}
        if append != "none":
            kw = dict(new_kv=(k_new.to(DEV), v_new.to(DEV)), rope_tables=rope_tables)
        out = _native.paged_decode(dq, k, v, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens),
                                   wl.head_dim**-0.5, seq_lens_host=host, **kw)
        return out, k, v

    fused = run()
    torch.cuda.synchronize()
    p1 = _native.decode_last_path()
    _native.set_decode_fused(False)
    passes = run()
    torch.cuda.synchronize()
    p2 = _native.decode_last_path()
    (o1, k1, v1), (o2, k2, v2) = fused, passes
    _log(f"  paths: {p1} / {p2}")
    assert p1 == "one_pass_merged" and p2 == "one_pass"
    assert _same_bits(o1, o2), "merge by the last split differs from the merge launch"
    assert _same_bits(k1, k2) and _same_bits(v1, v2)
    assert _control_regions_zero()
    if append == "none":
        err = (o1.cpu().float() - _decode_oracle(wl, kc, vc, q).float()).abs().max().item()
        _log(f"  max_abs_err={err:.3e}")
        assert err <= (2e-2 if dtype == torch.bfloat16 else 1e-4)


def test_one_pass_merge_by_last_split_back_to_back():
    """Many one-pass calls on one stream with no host synchronisation, long
    and short batches alternating (the merge by the last split forced on
    all of them): each equals its single-call result bit for bit, and the
    counters end zero."""
    _log("one-pass merged back to back")
    _native.set_attention_rounding("fast")
    _native.set_decode_fused(2)
    cases = [workloads.decode_ragged(seed=s) for s in (2, 4)] + [workloads.decode_small()]
    prepared = []
    for wl in cases:
        kc, vc = wl.pool(torch.bfloat16)
        q, _, _ = wl.new_tokens(torch.bfloat16)
        prepared.append((wl, kc.to(DEV), vc.to(DEV), q.to(DEV), torch.from_numpy(wl.table_array()).to(DEV),
                         torch.tensor(wl.seq_lens, dtype=torch.int32, device=DEV)))

    def call(p, host):
        wl, dk, dv, dq, tables, lens = p
        return _native.paged_decode(dq, dk, dv, 0, tables, lens, max(wl.seq_lens), sum(wl.seq_lens),
                                    wl.head_dim**-0.5, seq_lens_host=list(wl.seq_lens) if host else None)

    for host in (True, False):
        single = []
        for p in prepared:
            single.append(call(p, host))
            torch.cuda.synchronize()
            assert _native.decode_last_path() == "one_pass_merged"
        outs = [call(prepared[i % len(prepared)], host) for i in range(24)]
        torch.cuda.synchronize()
        for i, got in enumerate(outs):
            assert _same_bits(got, single[i % len(prepared)]), i
        assert _control_regions_zero()
