"""RMSNorm computed in fp32 and cast back (``layers/rms_norm.py:25-31`` of the reference)."""

import torch
from torch import nn

from nano_infer_engine import _native


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

    def _native_ok(self, x: torch.Tensor) -> bool:
        w = self.weight
        return x.is_cuda and _native.rms_norm_supported(x) and (
            w is None or (w.shape == (x.shape[-1],) and w.dtype == x.dtype and w.device == x.device))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._native_ok(x):
            # one HIP kernel (nie_rms_norm), the same arithmetic in fp32
            return _native.rms_norm(x, self.weight, self.eps)
        dtype = x.dtype
        h = x.float()
        h = h / torch.sqrt(torch.mean(torch.square(h), dim=-1, keepdim=True) + self.eps)
        if self.weight is not None:
            h = self.weight.float() * h
        return h.to(dtype)

    def forward_add(self, x: torch.Tensor, residual: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(x + residual, norm(x + residual)): the decoder's residual add before
        its post-attention norm (reference ``layers/decoder.py:50-51``), one
        kernel on the GPU."""
        if self._native_ok(x) and residual.shape == x.shape and residual.dtype == x.dtype and residual.is_cuda:
            return _native.rms_norm(x, self.weight, self.eps, residual=residual)
        h = x + residual
        return h, self.forward(h)
