"""SwiGLU feed-forward block (``layers/mlp.py:18-22`` of the reference)."""

import torch
import torch.nn.functional as F
from torch import nn

from nano_infer_engine import _native
from nano_infer_engine.layers import linear as _linear


class SwiGLUMLP(nn.Module):
    def __init__(self, inner_size: int, hidden_size: int):
        super().__init__()
        self.hidden_size = hidden_size
        self.inner_size = inner_size
        self.down_proj = nn.Linear(inner_size, hidden_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, inner_size, bias=False)
        self.gate_proj = nn.Linear(hidden_size, inner_size, bias=False)
        # [gate; up] weight rows for one projection GEMM on the GPU, rebuilt
        # whenever either weight is replaced or modified
        self._gate_up_weight: torch.Tensor | None = None
        self._gate_up_key: tuple | None = None

    def _stacked_gate_up_weight(self) -> torch.Tensor:
        ws = (self.gate_proj.weight, self.up_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        if key != self._gate_up_key:
            with torch.no_grad():
                self._gate_up_weight = torch.cat(ws, dim=0)
            self._gate_up_key = key
        return self._gate_up_weight

    def forward_normed(self, x, residual, norm):
        """``(self(norm(h)), h)`` for ``h = x + residual``, with the residual add
        and the norm folded into the gate/up GEMM and its SwiGLU epilogue (one
        launch for a decode step's rows), or None when the HIP path does not
        take the shapes."""
        ws = (self.gate_proj.weight, self.up_proj.weight)
        if (not x.is_cuda or ws[0].shape != ws[1].shape
                or any(p.bias is not None for p in (self.gate_proj, self.up_proj))
                or (torch.is_grad_enabled() and any(w.requires_grad for w in ws))):
            return None
        r = _linear.rms_norm_linear(x, residual, norm, self._stacked_gate_up_weight(), silu_mul=True)
        if r is None:
            return None
        h, act = r
        return _linear.apply(self.down_proj, act), h

    def forward(self, x):
        ws = (self.gate_proj.weight, self.up_proj.weight)
        if x.is_cuda and not (torch.is_grad_enabled() and any(w.requires_grad for w in ws)):
            # one GEMM over the concatenated weights (a captured decode graph
            # keeps the concatenation it was captured with), then
            # silu(gate) * up in one HIP kernel over the two halves
            self._stacked_gate_up_weight()
            if ws[0].shape == ws[1].shape:
                # a decode step's rows: both projections and the gated
                # product in one HIP GEMM
                h = _linear.silu_mul_linear(x, self._gate_up_weight, ws[0].shape[0])
                if h is not None:
                    return _linear.apply(self.down_proj, h)
            gate, up = F.linear(x, self._gate_up_weight).split((ws[0].shape[0], ws[1].shape[0]), dim=-1)
            if _native.silu_mul_supported(gate):
                return _linear.apply(self.down_proj, _native.silu_mul(gate, up))
            return _linear.apply(self.down_proj, F.silu(gate) * up)
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))
