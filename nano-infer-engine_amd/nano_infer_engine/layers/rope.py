"""Rotary position embeddings (plain and llama3-scaled).

Numerics follow ``layers/rope.py:6-200`` of the reference engine: inverse
frequencies and angles in fp32, sin/cos cast to the activation dtype, then
the rotate-half update ``(x1*cos - x2*sin, x2*cos + x1*sin)`` in the
activation dtype.  The inverse-frequency vector is computed once per device
instead of on every call, and :meth:`_RopeBase.tables` keeps per-position
sin/cos rows for the fused RoPE + KV-append kernel.
"""

from __future__ import annotations

import math

import torch
from torch import nn


def apply_rotary(x: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE; sin/cos broadcast over the head axis (dim -2)."""
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)


class _RopeBase(nn.Module):
    def __init__(self, dim: int, theta_base: float) -> None:
        super().__init__()
        if dim % 2:
            raise ValueError("RoPE dimension must be even")
        self.dim = dim
        self.theta_base = theta_base
        self._inv_freq: dict[torch.device, torch.Tensor] = {}
        self._tables: dict[tuple[torch.device, torch.dtype], tuple[torch.Tensor, torch.Tensor]] = {}

    def _compute_inv_freq(self, device: torch.device) -> torch.Tensor:
        exponents = torch.arange(0, self.dim, 2, dtype=torch.float32, device=device) / self.dim
        return 1 / self.theta_base**exponents

    def inv_freq(self, device: torch.device) -> torch.Tensor:
        cached = self._inv_freq.get(device)
        if cached is None:
            cached = self._compute_inv_freq(device)
            self._inv_freq[device] = cached
        return cached

    def sin_cos(self, positions: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        """sin/cos of shape positions.shape + (dim/2,), cast to ``dtype``."""
        angles = positions.to(torch.float32)[..., None] * self.inv_freq(positions.device)
        return torch.sin(angles).to(dtype), torch.cos(angles).to(dtype)

    def tables(self, device: torch.device, dtype: torch.dtype, rows: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(cos, sin) tables with at least ``rows`` rows: row p = cos/sin of p * inv_freq in ``dtype``.

        Built with the same torch ops as :meth:`sin_cos`, so row p equals
        ``sin_cos(p)`` bit for bit; the fused RoPE + KV-append kernel reads
        them.  Grown (and rebuilt) in steps of 4096 positions.
        """
        key = (device, dtype)
        cached = self._tables.get(key)
        if cached is None or cached[0].shape[0] < rows:
            size = max(4096, -(-rows // 4096) * 4096)
            positions = torch.arange(size, dtype=torch.int64, device=device)
            sin, cos = self.sin_cos(positions, dtype)
            cached = (cos.contiguous(), sin.contiguous())
            self._tables[key] = cached
        return cached

    def forward(self, x: torch.Tensor, position_offset: int = 0, position_ids: torch.Tensor | None = None):
        """x: (B, S, H, D).  Positions are offset..offset+S-1 or ``position_ids`` (B, S)."""
        bs, seq_len, _, head_dim = x.shape
        if head_dim != self.dim:
            raise ValueError(f"expected head_dim {self.dim}, got {head_dim}")
        if position_ids is None:
            positions = torch.arange(position_offset, position_offset + seq_len, device=x.device)[None]
        else:
            if position_ids.shape != (bs, seq_len):
                raise ValueError(f"position_ids must have shape {(bs, seq_len)}, got {tuple(position_ids.shape)}")
            positions = position_ids.to(x.device)
        sin, cos = self.sin_cos(positions, x.dtype)
        return apply_rotary(x, sin[:, :, None, :], cos[:, :, None, :])

    def rotate_tokens(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """x: (T, H, D) packed tokens at absolute ``positions`` (T,)."""
        sin, cos = self.sin_cos(positions, x.dtype)
        return apply_rotary(x, sin[:, None, :], cos[:, None, :])


class Rope(_RopeBase):
    """Unscaled RoPE (``rope_type="default"``)."""

    def __init__(self, dim: int, theta_base: float = 500000) -> None:
        super().__init__(dim, theta_base)


class RopeScale(_RopeBase):
    """Llama-3 frequency-banded RoPE scaling (``rope_type="llama3"``)."""

    def __init__(
        self,
        dim: int,
        theta_base: float = 500000.0,
        scaling_factor: float = 32.0,
        low_freq_factor: float = 1.0,
        high_freq_factor: float = 4.0,
        original_max_position_embeddings: int = 8192,
    ) -> None:
        super().__init__(dim, theta_base)
        self.scaling_factor = scaling_factor
        self.low_freq_factor = low_freq_factor
        self.high_freq_factor = high_freq_factor
        self.original_max_position_embeddings = original_max_position_embeddings

    def _compute_inv_freq(self, device: torch.device) -> torch.Tensor:
        base = super()._compute_inv_freq(device)
        wavelength = 2 * math.pi / base
        old_ctx = self.original_max_position_embeddings
        # long wavelengths are slowed down by the scaling factor, short ones
        # kept, and the band in between interpolated linearly in 1/wavelength
        slowed = base / self.scaling_factor
        blend = (old_ctx / wavelength - self.low_freq_factor) / (self.high_freq_factor - self.low_freq_factor)
        interpolated = (1 - blend) * slowed + blend * base
        low = wavelength > old_ctx / self.low_freq_factor
        high = wavelength < old_ctx / self.high_freq_factor
        out = torch.where(low, slowed, base)
        return torch.where(~(low | high), interpolated, out)
