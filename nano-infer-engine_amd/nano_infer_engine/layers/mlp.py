"""SwiGLU feed-forward block (``layers/mlp.py:18-22`` of the reference)."""

import torch.nn.functional as F
from torch import nn

from nano_infer_engine import _native


class SwiGLUMLP(nn.Module):
    def __init__(self, inner_size: int, hidden_size: int):
        super().__init__()
        self.hidden_size = hidden_size
        self.inner_size = inner_size
        self.down_proj = nn.Linear(inner_size, hidden_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, inner_size, bias=False)
        self.gate_proj = nn.Linear(hidden_size, inner_size, bias=False)

    def forward(self, x):
        gate, up = self.gate_proj(x), self.up_proj(x)
        if gate.is_cuda and _native.silu_mul_supported(gate):
            # silu(gate) * up in one HIP kernel (nie_silu_mul), torch's roundings
            return self.down_proj(_native.silu_mul(gate, up))
        return self.down_proj(F.silu(gate) * up)
