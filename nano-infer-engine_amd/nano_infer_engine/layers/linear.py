"""Bias-free projections of the decoder: ``nn.Linear``, optionally a decode step's rows on nie_linear_rows.

The reference engine runs every projection as ``nn.Linear`` (``layers/attention.py:227-232``,
``:271``, ``:359-361``, ``:414``; ``layers/mlp.py:18-22``; ``models/llama.py:328``, ``:391``).
By default this build does the same: torch's GEMM gives the reference's results bit for bit
(the stacked [q; k; v] and [gate; up] products included: each output element is the same
dot product in the same library kernel), which the bf16 serving identity needs.
``nie_linear_rows`` streams a decode step's weights faster (up to 16 bf16 rows) but
accumulates in another order: about 1.6e-4 of its bf16 outputs differ by one ulp from
torch's, enough to move the serving lockstep's agreement with the reference path from
95% to 94%.  ``USE_NATIVE = True`` opts in to it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nano_infer_engine import _native

#: Route eligible projections to nie_linear_rows (off: torch's GEMM, the
#: reference's arithmetic).
USE_NATIVE = False


#: Tiles of 16 output columns that keep every CU streaming: the kernel runs
#: one workgroup per CU over its tiles, so a weight with fewer tiles and a long
#: inner dimension (SwiGLU's down projection: 128 tiles, k = 8192) leaves half
#: the GPU idle and is faster on torch's split-k GEMM (13 us against 17 us).
_FULL_GRID_TILES = 256


def _native_ok(x: torch.Tensor, weight: torch.Tensor, silu_mul: bool = False) -> bool:
    if not USE_NATIVE or not _native.linear_rows_supported(x, weight, silu_mul):
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
    if gate_up_weight.shape[0] != 2 * inner or not _native_ok(x, gate_up_weight, silu_mul=True) or inner % 16:
        return None
    return _native.linear_rows(x, gate_up_weight, silu_mul=True)


def rms_norm_linear(x: torch.Tensor, residual: torch.Tensor | None, norm: nn.Module, weight: torch.Tensor,
                    silu_mul: bool = False, want_sum: bool = True):
    """``(x + residual, linear(norm(x + residual), weight))`` in one launch
    (``silu_mul``: the SwiGLU product of a stacked ``[gate; up]`` weight), or
    None when the HIP path does not take the shapes.  ``norm`` is an
    ``RmsNorm`` with a weight; the sum is None without a residual.

    Not while a HIP graph is being captured: the folded norm saves a launch,
    but each of the GEMM's workgroups reads x and the residual again (128 KiB
    each), which costs more GPU time than the separate norm kernel once
    launches are replayed from a graph (8273 against 7812 output tok/s on the
    serving workload); launched one by one (eager steps: 5410 against 4296)
    the saved launch wins."""
    if torch.cuda.is_current_stream_capturing():
        return None
    nw = getattr(norm, "weight", None)
    if nw is None or nw.shape != (x.shape[-1],) or nw.dtype != x.dtype or nw.device != x.device:
        return None
    if (weight.ndim != 2 or weight.shape[1] != _native.RMS_NORM_LINEAR_K
            or not _native_ok(x, weight, silu_mul=silu_mul)):
        return None
    if torch.is_grad_enabled() and nw.requires_grad:
        return None
    if residual is not None and (residual.shape != x.shape or residual.dtype != x.dtype
                                 or residual.device != x.device):
        return None
    if silu_mul and weight.shape[0] % 32:
        return None
    return _native.rms_norm_linear_rows(x, residual, nw, norm.eps, weight, silu_mul=silu_mul, want_sum=want_sum)
