"""Writes the golden fixtures of the paged-attention path (run from the repo root).

    python tests/golden/make_golden.py

Each fixture holds the float64 closed-form attention (textbook softmax
attention with the GQA map h -> h // (Hq/Hkv) and the causal position mask)
of a seeded workload, stored as float32, plus a SHA-256 fingerprint of the
inputs so a test notices if the seeded generator ever produces different
values.  Inputs are not stored: they are regenerated from the seed by
``nano_infer_engine.workloads``.

Fixtures
  decode_small_{f32,bf16}.npz   4 decode rows of {17, 64, 129, 500} tokens,
                                32 q / 8 kv heads, head_dim 64, block 16
  ragged_small_{f32,bf16}.npz   5 requests, contexts {0, 3, 50, 0, 17},
                                new tokens {19, 5, 1, 40, 2}, 4 q / 2 kv
                                heads, head_dim 64, block 16
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(REPO, "nano-infer-engine_amd"), REPO]

from nano_infer_engine import workloads  # noqa: E402
from oracle import closed_form, reference_ops  # noqa: E402

DTYPES = {"f32": torch.float32, "bf16": torch.bfloat16}


def fingerprint(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.float().contiguous().numpy().tobytes())
    return h.hexdigest()


def decode_small_workload():
    return workloads.decode_small()


def ragged_small_workload():
    return workloads.ragged([0, 3, 50, 0, 17], [19, 5, 1, 40, 2], seed=13, pool_factor=1.5, q_heads=4, kv_heads=2,
                            head_dim=64, block_size=16)


def decode_expected(wl, dtype):
    kc, vc = wl.pool(dtype)
    q, _, _ = wl.new_tokens(dtype)
    out = np.zeros((len(wl.seq_lens), wl.q_heads, wl.head_dim))
    for b, n in enumerate(wl.seq_lens):
        ks, vs = reference_ops.gather_tokens(kc, vc, 0, wl.tables[b], wl.block_size, n)
        out[b] = closed_form.decode(q[b].double().numpy(), ks.double().numpy(), vs.double().numpy(), wl.head_dim**-0.5)
    return out.astype(np.float32), fingerprint(q, kc, vc)


def ragged_expected(wl, dtype):
    kc, vc = wl.pool(dtype)
    q, k, v = wl.new_tokens(dtype)
    keys, values = kc.clone(), vc.clone()
    out, start = [], 0
    for table, c, n in zip(wl.tables, wl.context_lens, wl.query_lens):
        reference_ops.write_tokens(keys, values, 0, table, wl.block_size, c, k[start : start + n], v[start : start + n])
        ks, vs = reference_ops.gather_tokens(keys, values, 0, table, wl.block_size, c + n)
        out.append(closed_form.attention(q[start : start + n].double().numpy(), ks.double().numpy(),
                                         vs.double().numpy(), list(range(c, c + n)), wl.head_dim**-0.5))
        start += n
    return np.concatenate(out).astype(np.float32), fingerprint(q, k, v, kc, vc)


def main():
    for tag, dtype in DTYPES.items():
        exp, fp = decode_expected(decode_small_workload(), dtype)
        np.savez_compressed(os.path.join(HERE, f"decode_small_{tag}.npz"), expected=exp, fingerprint=np.array(fp))
        exp, fp = ragged_expected(ragged_small_workload(), dtype)
        np.savez_compressed(os.path.join(HERE, f"ragged_small_{tag}.npz"), expected=exp, fingerprint=np.array(fp))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
