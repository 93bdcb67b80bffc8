"""RMSNorm computed in fp32 and cast back (``layers/rms_norm.py:25-31`` of the reference)."""

import torch
from torch import nn


class RmsNorm(nn.Module):
    def __init__(self, normalized_shape, eps: float = 1e-5, elementwise_affine: bool = True, device=None, dtype=None):
        super().__init__()
        self.eps = eps
        self.normalized_shape = normalized_shape
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(normalized_shape, device=device, dtype=dtype))
        else:
            self.register_parameter("weight", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dtype = x.dtype
        h = x.float()
        h = h / torch.sqrt(torch.mean(torch.square(h), dim=-1, keepdim=True) + self.eps)
        if self.weight is not None:
            h = self.weight.float() * h
        return h.to(dtype)
