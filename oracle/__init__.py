"""Oracle for the paged-attention path — TEST INFRASTRUCTURE ONLY.

This package restates the reference engine's algorithm for the hot path
(ito-integral/nano-infer-engine, torch ops in Python loops) so the HIP
kernels can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
it, and only as the checker or the timed CPU baseline.  The product package
(``nano_infer_engine``) never imports it and has no CPU fallback.

Modules
  reference_ops    per-block decode attention, per-token KV write/gather,
                   per-request ragged attention — loop-for-loop restatements
                   of the reference (file:line cited on each function)
  closed_form      float64 numpy attention over contiguous K/V (textbook
                   softmax attention with GQA and a causal position mask)
  slots            closed-form slot mapping / block-table arithmetic (numpy)

How each function is pinned (see tests/test_oracle.py):
  * slot math, write/gather   — the reference tests' known answers
    (block counts (1,1),(4,1),(5,2),(8,2),(9,3); fragmented table (2, 0);
    allocator order [0, 1] and reuse order) and bit-exact round trips;
  * decode attention           — float64 closed form, plus invariants that a
    dropped term / wrong GQA index / wrong block order would break
    (length-1 sequence returns V exactly, equal keys average V, permuting
    physical blocks is bit-identical, garbage past the length is ignored);
  * ragged attention           — float64 closed form with the causal offset,
    chunked == one-shot, a length-1 row equals decode at length ctx+1.
  * bf16 rounding points       — checked against float64 within bf16
    tolerance only: torch's internal accumulation order inside
    einsum/matmul is not pinned bit-for-bit ("parity unpinned" at the bit
    level for bf16; the tolerance contract is max-abs <= 2e-2).
"""
