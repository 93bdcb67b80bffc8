"""SwiGLU feed-forward block (``layers/mlp.py:18-22`` of the reference)."""

import torch.nn.functional as F
from torch import nn


class SwiGLUMLP(nn.Module):
    def __init__(self, inner_size: int, hidden_size: int):
        super().__init__()
        self.hidden_size = hidden_size
        self.inner_size = inner_size
        self.down_proj = nn.Linear(inner_size, hidden_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, inner_size, bias=False)
        self.gate_proj = nn.Linear(hidden_size, inner_size, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))
