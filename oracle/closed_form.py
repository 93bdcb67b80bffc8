"""Float64 closed-form attention (numpy).  Test infrastructure only.

Textbook scaled-dot-product attention with grouped-query heads: query head h
reads KV head h // (Hq / Hkv) — the mapping ``repeat_interleave(G, dim=1)``
produces in the reference (``layers/paged_attention.py:92-93``,
``layers/attention.py:395-396``) — and key position j is visible to a query
at position p iff j <= p (``layers/attention.py:401-409``).
"""

from __future__ import annotations

import numpy as np


def attention(q, k, v, q_positions, scale: float) -> np.ndarray:
    """q (Tq, Hq, D), k/v (S, Hkv, D), q_positions (Tq,) -> (Tq, Hq, D) float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    tq, hq, d = q.shape
    s, hkv, _ = k.shape
    group = hq // hkv
    out = np.zeros((tq, hq, d), dtype=np.float64)
    key_pos = np.arange(s)
    for h in range(hq):
        kh = k[:, h // group, :]
        vh = v[:, h // group, :]
        scores = (q[:, h, :] @ kh.T) * scale  # (Tq, S)
        visible = key_pos[None, :] <= np.asarray(q_positions)[:, None]
        scores = np.where(visible, scores, -np.inf)
        scores = scores - scores.max(axis=1, keepdims=True)
        w = np.exp(scores)
        w /= w.sum(axis=1, keepdims=True)
        out[:, h, :] = w @ vh
    return out


def decode(q, k, v, scale: float) -> np.ndarray:
    """One query per head (Hq, D) over all S keys -> (Hq, D)."""
    k = np.asarray(k)
    return attention(np.asarray(q)[None], k, v, [k.shape[0] - 1], scale)[0]
