"""Grouped-query attention over the paged KV cache.

Public surface of ``GroupedQueryAttention`` in ``layers/attention.py:121-414``
of the reference engine: the constructor, ``forward`` with its paged decode
branch (``paged_cache=``, ``layer_index=``, ``sequence_id=``,
``sequence_ids=``; same checks and messages) and ``forward_ragged``.  The
projections run through :mod:`layers.linear` (the HIP GEMM for a decode
step's rows, torch's otherwise); RoPE, the K/V write and
the attention itself go through :data:`attention_core`
(:func:`paged_batch.attention_core`: one fused RoPE + KV-append launch plus
the decode / varlen-prefill kernels).

Both methods take an optional ``paged_batch`` — the per-forward metadata the
model builds once for all layers.  Without it they build their own, so the
reference's call pattern still works.

Dense (contiguous-cache) attention is not part of this build.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from nano_infer_engine.layers import linear as _linear
from nano_infer_engine.layers.rope import Rope
from nano_infer_engine import paged_batch as _paged_batch
from nano_infer_engine.paged_batch import RaggedBatch, build_ragged_batch
from nano_infer_engine.paged_cache import PagedKVCache

#: Per-layer attention core: (q, k, v, cache, layer_index, batch, scale, rope)
#: -> context, with q/k not yet rotated.  Module-level so a caller can swap
#: in another implementation of the same contract.
attention_core = _paged_batch.attention_core


class GroupedQueryAttention(nn.Module):
    def __init__(self, q_head_num: int, kv_head_num: int, hidden_size: int, rope=None):
        super().__init__()
        assert hidden_size % q_head_num == 0
        assert q_head_num % kv_head_num == 0
        self.head_dim = hidden_size // q_head_num
        self.q_head_num = q_head_num
        self.kv_head_num = kv_head_num
        self.hidden_size = hidden_size
        self.group_num = q_head_num // kv_head_num
        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.k_proj = nn.Linear(hidden_size, kv_head_num * self.head_dim, bias=False)
        self.v_proj = nn.Linear(hidden_size, kv_head_num * self.head_dim, bias=False)
        self.o_proj = nn.Linear(hidden_size, hidden_size, bias=False)
        self.rope = Rope(self.head_dim) if rope is None else rope
        # [q; k; v] weight rows for one projection GEMM on the GPU, rebuilt
        # whenever one of the three weights is replaced or modified
        self._qkv_weight: torch.Tensor | None = None
        self._qkv_key: tuple | None = None

    def _project_qkv(self, x: torch.Tensor):
        """q, k, v = q_proj(x), k_proj(x), v_proj(x) (``layers/attention.py:227-238``, ``:359-361``).

        On the GPU without autograd this is one GEMM over the concatenated
        weights; q, k and v are then column slices of its output.  A captured
        decode graph keeps the concatenation it was captured with (weights
        changed afterwards need a new capture, as any captured weight would).
        """
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        if not x.is_cuda or (torch.is_grad_enabled() and any(w.requires_grad for w in ws)):
            return self.q_proj(x), self.k_proj(x), self.v_proj(x)
        qkv = _linear.linear(x, self._stacked_qkv_weight())
        return qkv.split((ws[0].shape[0], ws[1].shape[0], ws[2].shape[0]), dim=-1)

    def _stacked_qkv_weight(self) -> torch.Tensor:
        """[q; k; v] weight rows, rebuilt whenever one of them changes."""
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype, w.device) for w in ws)
        if key != self._qkv_key:
            with torch.no_grad():
                self._qkv_weight = torch.cat(ws, dim=0)
            self._qkv_key = key
        return self._qkv_weight

    def project_qkv_normed(self, x: torch.Tensor, residual: torch.Tensor | None, norm: nn.Module):
        """``h = x + residual`` (``x`` without one), then q, k, v of ``norm(h)``:
        the pre-attention norm folded into the projection GEMM (one launch for
        a decode step's rows).  Returns ``(h, q, k, v)``, or None when the HIP
        path does not take the shapes (callers then norm and project apart)."""
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight)
        if (not x.is_cuda or any(p.bias is not None for p in (self.q_proj, self.k_proj, self.v_proj))
                or (torch.is_grad_enabled() and any(w.requires_grad for w in ws))):
            return None
        r = _linear.rms_norm_linear(x, residual, norm, self._stacked_qkv_weight())
        if r is None:
            return None
        h, qkv = r
        q, k, v = qkv.split((ws[0].shape[0], ws[1].shape[0], ws[2].shape[0]), dim=-1)
        return (x if h is None else h), q, k, v

    # ------------------------------------------------------------------
    def forward_tokens(
        self,
        x: torch.Tensor,
        paged_cache: PagedKVCache,
        layer_index: int,
        batch: RaggedBatch,
        *,
        qkv: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    ) -> torch.Tensor:
        """Attention for packed tokens x (num_tokens, hidden) described by ``batch``.

        ``qkv``: the tokens' projections, already computed (``x`` is then unused).
        """
        q, k, v = self._project_qkv(x) if qkv is None else qkv
        tokens = q.shape[0]
        q = q.view(tokens, self.q_head_num, self.head_dim)
        k = k.view(tokens, self.kv_head_num, self.head_dim)
        v = v.view(tokens, self.kv_head_num, self.head_dim)
        context = attention_core(q, k, v, paged_cache, layer_index, batch, self.head_dim**-0.5, self.rope)
        return _linear.apply(self.o_proj, context.view(tokens, self.hidden_size))

    def forward(
        self,
        x,
        k_cache=None,
        v_cache=None,
        cache_position=0,
        attention_mask=None,
        position_ids=None,
        *,
        paged_cache: PagedKVCache | None = None,
        layer_index: int | None = None,
        sequence_id: str = "default",
        sequence_ids: tuple[str, ...] | None = None,
        paged_batch: RaggedBatch | None = None,
    ):
        """Paged decode step: x (batch, 1, hidden) -> (batch, 1, hidden).

        Each sequence's new K/V goes to position ``cached length`` and the
        query attends to ``cached length + 1`` tokens
        (``layers/attention.py:178-273`` of the reference).
        """
        bs, seq_len, hidden_size = x.shape
        assert hidden_size == self.hidden_size
        if (k_cache is None) != (v_cache is None):
            raise ValueError("k_cache and v_cache must both be provided or both be None")
        if paged_cache is not None and (k_cache is not None or v_cache is not None):
            raise ValueError("contiguous cache and paged cache cannot be used together")
        if paged_cache is None:
            raise NotImplementedError("this build implements attention over a PagedKVCache only")
        if seq_len != 1:
            raise ValueError("paged attention reference currently requires seq_len=1")
        if layer_index is None:
            raise ValueError("layer_index is required for paged attention")
        if attention_mask is not None and not bool(attention_mask.all()):
            raise ValueError("paged attention reference does not support padding masks")
        if sequence_ids is None:
            if bs != 1:
                raise ValueError("sequence_ids is required for batched paged attention")
            ids: tuple[str, ...] = (sequence_id,)
        else:
            if not isinstance(sequence_ids, tuple):
                raise TypeError("sequence_ids must be a tuple")
            if len(sequence_ids) != bs:
                raise ValueError("sequence_ids must match the batch size")
            if any(not isinstance(s, str) or not s for s in sequence_ids):
                raise ValueError("sequence IDs must be non-empty strings")
            if len(set(sequence_ids)) != len(sequence_ids):
                raise ValueError("sequence IDs must be unique within a batch")
            ids = sequence_ids
        lengths = tuple(paged_cache.get_sequence_length(s) for s in ids)
        if position_ids is not None:
            expected = torch.tensor(lengths, dtype=torch.long, device=x.device)[:, None]
            if not torch.equal(position_ids, expected):
                raise ValueError("position_ids must match paged cache sequence lengths")
        if paged_batch is None:
            paged_batch = build_ragged_batch(paged_cache, ids, (1,) * bs, lengths)
        out = self.forward_tokens(x.reshape(bs, hidden_size), paged_cache, layer_index, paged_batch)
        return out.view(bs, 1, hidden_size)

    def forward_ragged(
        self,
        x: torch.Tensor,
        *,
        paged_cache: PagedKVCache,
        layer_index: int,
        sequence_ids: tuple[str, ...],
        query_start_loc: torch.Tensor,
        context_lengths: tuple[int, ...],
        paged_batch: RaggedBatch | None = None,
    ) -> torch.Tensor:
        """Flattened variable-length chunks x (total_tokens, hidden) -> (total_tokens, hidden).

        Request r owns rows query_start_loc[r]..query_start_loc[r+1]-1 at
        positions context_lengths[r] + i: causal inside its chunk, full
        attention to its cached prefix (``layers/attention.py:345-414``).
        """
        total_tokens, hidden_size = x.shape
        assert hidden_size == self.hidden_size
        if paged_batch is None:
            bounds = query_start_loc.tolist()
            query_lens = tuple(b - a for a, b in zip(bounds, bounds[1:]))
            paged_batch = build_ragged_batch(paged_cache, tuple(sequence_ids), query_lens, tuple(context_lengths))
        return self.forward_tokens(x, paged_cache, layer_index, paged_batch)
