"""Bias-free projections of the decoder: ``nn.Linear`` for a decode step's rows on nie_linear_rows.

The reference engine runs every projection as ``nn.Linear`` (``layers/attention.py:227-232``,
``:271``, ``:359-361``, ``:414``; ``layers/mlp.py:18-22``; ``models/llama.py:328``, ``:391``).
A decode step multiplies at most one row per sequence by each weight, which torch's
library GEMM handles at a small fraction of the HBM bandwidth; up to 16 bf16 rows go
to the HIP kernel, everything else (prefill chunks, fp32, autograd) stays with torch.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nano_infer_engine import _native

#: Route eligible projections to nie_linear_rows (tests switch it off to
#: compare against torch's GEMM).
USE_NATIVE = True


#: Tiles of 16 output columns that keep every CU streaming: the kernel runs
#: one workgroup per CU over its tiles, so a weight with fewer tiles and a long
#: inner dimension (SwiGLU's down projection: 128 tiles, k = 8192) leaves half
#: the GPU idle and is faster on torch's split-k GEMM (13 us against 17 us).
_FULL_GRID_TILES = 256


def _native_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    if not USE_NATIVE or not _native.linear_rows_supported(x, weight):
        return False
    n, k = weight.shape
    if k > 4096 and n // 16 < _FULL_GRID_TILES:
        return False
    return not (torch.is_grad_enabled() and (weight.requires_grad or x.requires_grad))


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, weight)`` without a bias."""
    if _native_ok(x, weight):
        return _native.linear_rows(x, weight)
    return F.linear(x, weight)


def apply(module: nn.Linear, x: torch.Tensor) -> torch.Tensor:
    """``module(x)`` for an ``nn.Linear``; bias-free ones may take the HIP path."""
    if module.bias is None:
        return linear(x, module.weight)
    return module(x)


def silu_mul_linear(x: torch.Tensor, gate_up_weight: torch.Tensor, inner: int) -> torch.Tensor | None:
    """``silu(x . Wg^T) * (x . Wu^T)`` from the stacked ``[gate; up]`` weight in one
    launch, or None when the HIP path does not take the shapes."""
    if gate_up_weight.shape[0] != 2 * inner or not _native_ok(x, gate_up_weight) or inner % 16:
        return None
    return _native.linear_rows(x, gate_up_weight, silu_mul=True)
