"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the seeded inputs still fingerprint the same, and the oracle's
restatement of the reference algorithm lands on the float64 fixture within
its dtype's tolerance.  GPU: the HIP kernels, called through the C ABI,
land on the same fixture (fp32 max-abs <= 1e-4, bf16 <= 2e-2).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from nano_infer_engine import _native

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_golden  # noqa: E402
from oracle import reference_ops  # noqa: E402

TOL = {"f32": 1e-4, "bf16": 2e-2}
ORACLE_TOL = {"f32": 1e-5, "bf16": 2e-2}


def _fixture(name):
    data = np.load(os.path.join(HERE, name + ".npz"))
    return data["expected"], str(data["fingerprint"])


def _decode_inputs(tag):
    wl = make_golden.decode_small_workload()
    kc, vc = wl.pool(make_golden.DTYPES[tag])
    q, _, _ = wl.new_tokens(make_golden.DTYPES[tag])
    return wl, kc, vc, q


def _ragged_inputs(tag):
    wl = make_golden.ragged_small_workload()
    kc, vc = wl.pool(make_golden.DTYPES[tag])
    q, k, v = wl.new_tokens(make_golden.DTYPES[tag])
    return wl, kc, vc, q, k, v


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_oracle_decode_matches_fixture(tag):
    expected, fp = _fixture(f"decode_small_{tag}")
    wl, kc, vc, q = _decode_inputs(tag)
    assert make_golden.fingerprint(q, kc, vc) == fp
    got = reference_ops.batched_paged_attention_reference(q, kc, vc, tuple(tuple(t) for t in wl.tables),
                                                          tuple(wl.seq_lens), 0)
    assert np.abs(got.float().numpy() - expected).max() <= ORACLE_TOL[tag]


@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_oracle_ragged_matches_fixture(tag):
    expected, fp = _fixture(f"ragged_small_{tag}")
    wl, kc, vc, q, k, v = _ragged_inputs(tag)
    assert make_golden.fingerprint(q, k, v, kc, vc) == fp
    got = reference_ops.ragged_attention_reference(q, k, v, kc, vc, 0, wl.tables, wl.context_lens, wl.query_lens,
                                                   wl.head_dim**-0.5)
    assert np.abs(got.float().numpy() - expected).max() <= ORACLE_TOL[tag]


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_hip_decode_matches_fixture(tag):
    print(f"golden decode_small {tag}", flush=True)
    expected, _ = _fixture(f"decode_small_{tag}")
    wl, kc, vc, q = _decode_inputs(tag)
    dev = torch.device("cuda:0")
    tables = torch.from_numpy(wl.table_array()).to(dev)
    lens = torch.tensor(wl.seq_lens, dtype=torch.int32, device=dev)
    out = _native.paged_decode(q.to(dev), kc.to(dev), vc.to(dev), 0, tables, lens, max(wl.seq_lens),
                               sum(wl.seq_lens), wl.head_dim**-0.5)
    assert np.abs(out.float().cpu().numpy() - expected).max() <= TOL[tag]


@pytest.mark.gpu
@pytest.mark.parametrize("tag", ["f32", "bf16"])
def test_hip_ragged_matches_fixture(tag):
    print(f"golden ragged_small {tag}", flush=True)
    expected, _ = _fixture(f"ragged_small_{tag}")
    wl, kc, vc, q, k, v = _ragged_inputs(tag)
    dev = torch.device("cuda:0")
    dk, dv = kc.to(dev), vc.to(dev)
    _native.kv_append(dk, dv, 0, k.to(dev), v.to(dev), torch.from_numpy(wl.slots()).to(dev))
    cu = torch.tensor(np.concatenate([[0], np.cumsum(wl.query_lens)]), dtype=torch.int64, device=dev)
    ctx = torch.tensor(wl.context_lens, dtype=torch.int32, device=dev)
    tables = torch.from_numpy(wl.table_array()).to(dev)
    out = _native.varlen_prefill(q.to(dev), cu, ctx, dk, dv, 0, tables, max(wl.query_lens), max(wl.seq_lens),
                                 wl.head_dim**-0.5)
    assert np.abs(out.float().cpu().numpy() - expected).max() <= TOL[tag]
