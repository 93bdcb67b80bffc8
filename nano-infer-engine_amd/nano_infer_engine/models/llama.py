"""Llama-3.2 decoder-only model over the paged KV cache.

Configuration and module layout follow ``models/llama.py:14-394`` of the
reference engine (same ``LlamaConfig`` fields and defaults, same parameter
names, so state dicts are interchangeable).  ``forward`` (paged decode and
equal-length paged prefill) and ``forward_ragged`` keep the reference's
signatures and checks; both build one :class:`RaggedBatch` per call and run
every layer on packed tokens, so the per-layer attention is one KV-append
launch plus the HIP decode / varlen-prefill kernels.

Calling ``forward`` without a cache runs the same path over a temporary
paged cache (full causal attention over the input).  The dense ``KVCache``
of the reference is not part of this build.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch import nn

from nano_infer_engine import _native
from nano_infer_engine.layers import linear as _linear
from nano_infer_engine.layers.decoder import Llama3Decoder
from nano_infer_engine.layers.rms_norm import RmsNorm
from nano_infer_engine.layers.rope import Rope, RopeScale
from nano_infer_engine.paged_batch import RaggedBatch, build_ragged_batch
from nano_infer_engine.paged_cache import PagedKVCache


@dataclass
class RopeScalingConfig:
    factor: float = 32.0
    low_freq_factor: float = 1.0
    high_freq_factor: float = 4.0
    original_max_position_embeddings: int = 8192


@dataclass
class LlamaConfig:
    vocab_size: int = 128256
    hidden_size: int = 2048
    mlp_inner_size: int = 8192
    num_layers: int = 16
    q_head_num: int = 32
    kv_head_num: int = 8
    norm_eps: float = 1e-5
    rope_type: str = "llama3"
    rope_theta: float = 500000.0
    max_seq_len: int = 131072
    rope_scaling: RopeScalingConfig = field(default_factory=RopeScalingConfig)
    hidden_act: str = "silu"
    attention_bias: bool = False
    mlp_bias: bool = False
    attention_dropout: float = 0.0
    tie_word_embeddings: bool = True
    initializer_range: float = 0.02
    bos_token_id: int = 128000
    eos_token_id: int = 128001

    def __post_init__(self):
        assert self.hidden_size % self.q_head_num == 0
        assert self.q_head_num % self.kv_head_num == 0
        assert self.head_dim % 2 == 0

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.q_head_num

    @property
    def group_num(self) -> int:
        return self.q_head_num // self.kv_head_num


def build_rope(config: LlamaConfig):
    if config.rope_type == "default":
        return Rope(dim=config.head_dim, theta_base=config.rope_theta)
    if config.rope_type == "llama3":
        s = config.rope_scaling
        return RopeScale(
            dim=config.head_dim,
            theta_base=config.rope_theta,
            scaling_factor=s.factor,
            low_freq_factor=s.low_freq_factor,
            high_freq_factor=s.high_freq_factor,
            original_max_position_embeddings=s.original_max_position_embeddings,
        )
    raise ValueError(f"Unsupported rope type: {config.rope_type}")


def _check_sequence_ids(sequence_ids, batch_size: int) -> None:
    if not isinstance(sequence_ids, tuple):
        raise TypeError("sequence_ids must be a tuple")
    if len(sequence_ids) != batch_size:
        raise ValueError("sequence_ids must match the batch size")
    if any(not isinstance(s, str) or not s for s in sequence_ids):
        raise ValueError("sequence IDs must be non-empty strings")
    if len(set(sequence_ids)) != len(sequence_ids):
        raise ValueError("sequence IDs must be unique within a batch")


class Llama3_2(nn.Module):
    def __init__(self, config: LlamaConfig):
        super().__init__()
        self.config = config
        self.embed = nn.Embedding(config.vocab_size, config.hidden_size)
        self.rope = build_rope(config)
        self.decoders = nn.ModuleList(
            Llama3Decoder(
                config.norm_eps,
                config.q_head_num,
                config.kv_head_num,
                config.hidden_size,
                config.mlp_inner_size,
                self.rope,
            )
            for _ in range(config.num_layers)
        )
        self.final_rms = RmsNorm(config.hidden_size, config.norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.embed.weight

    # ------------------------------------------------------------------
    def run_tokens(
        self,
        input_ids: torch.Tensor,
        cache: PagedKVCache,
        batch: RaggedBatch,
        logits_rows: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Embed packed tokens, run every layer over ``batch``, return logits.

        With ``logits_rows`` only those token rows go through the final norm
        and the LM head.
        """
        x = self.embed(input_ids)
        # each block's output stays an unsummed pair (ffn_out, h); the next
        # norm adds it (one kernel for the add and the norm on the GPU)
        lean = self._lean_stream(x)
        for layer_index, decoder in enumerate(self.decoders):
            if lean is not None:
                x = decoder.forward_tokens_lean(x, cache, layer_index, batch, lean)
            else:
                x = decoder.forward_tokens_unsummed(x, cache, layer_index, batch)
        if not isinstance(x, tuple):  # no layers
            x = (x, torch.zeros_like(x))
        ffn_out, h = x
        if logits_rows is not None:
            ffn_out, h = ffn_out[logits_rows], h[logits_rows]
        if self.lm_head.bias is None:
            # a decode step's rows: the final norm and its residual add inside
            # the LM-head GEMM
            r = _linear.rms_norm_linear(ffn_out, h, self.final_rms, self.lm_head.weight, want_sum=False)
            if r is not None:
                return r[1]
        return _linear.apply(self.lm_head, self.final_rms.forward_add(ffn_out, h)[1])

    def _lean_stream(self, x: torch.Tensor) -> int | None:
        """The current stream when every block can run ``forward_tokens_lean``
        on x's rows, else None: a packed batch of more than the decode-step
        GEMM's rows (a prefill step's; fewer rows keep the fused decode-step
        kernels), on the GPU, without autograd."""
        if (not x.is_cuda or x.dim() != 2 or x.shape[0] <= _native.LINEAR_MAX_ROWS or not x.is_contiguous()
                or torch.is_grad_enabled()):
            return None
        if not all(decoder.lean_weights(x) for decoder in self.decoders):
            return None
        return _native._stream(x.device)

    def _new_cache_for(self, batch_size: int, seq_len: int, device: torch.device) -> tuple[PagedKVCache, tuple[str, ...]]:
        block_size = 16
        per_seq = -(-seq_len // block_size)
        cache = PagedKVCache(
            num_blocks=batch_size * per_seq,
            block_size=block_size,
            num_layers=self.config.num_layers,
            kv_head_num=self.config.kv_head_num,
            head_dim=self.config.head_dim,
            dtype=self.embed.weight.dtype,
            device=device,
        )
        return cache, tuple(f"sequence-{i}" for i in range(batch_size))

    def forward(
        self,
        x: torch.Tensor,
        kv_cache: PagedKVCache | None = None,
        attention_mask: torch.Tensor | None = None,
        position_ids: torch.Tensor | None = None,
        sequence_id: str = "default",
        sequence_ids: tuple[str, ...] | None = None,
    ) -> torch.Tensor:
        """x (batch, seq_len) token IDs -> logits (batch, seq_len, vocab)."""
        batch_size, seq_len = x.shape
        if kv_cache is None:
            if attention_mask is not None and not bool(attention_mask.bool().all()):
                raise ValueError("padding masks are not supported by this build")
            cache, ids = self._new_cache_for(batch_size, seq_len, x.device)
            return self.forward(x, kv_cache=cache, position_ids=position_ids, sequence_ids=ids)
        if not isinstance(kv_cache, PagedKVCache):
            raise TypeError("this build runs the model over a PagedKVCache only")

        decode = seq_len == 1
        if sequence_ids is None:
            if batch_size != 1:
                raise ValueError("sequence_ids is required for batched paged inference")
            ids = (sequence_id,)
        else:
            _check_sequence_ids(sequence_ids, batch_size)
            ids = sequence_ids
        lengths = tuple(kv_cache.get_sequence_length(s) for s in ids)
        if not decode and len(set(lengths)) != 1:
            raise ValueError("batched paged prefill currently requires equal sequence lengths")
        total_seq_len = (max(lengths) + 1) if decode else lengths[0] + seq_len
        if total_seq_len > self.config.max_seq_len:
            raise ValueError(f"Sequence length {total_seq_len} exceeds max_seq_len={self.config.max_seq_len}")
        for s, length in zip(ids, lengths):
            kv_cache.ensure_capacity(s, length + seq_len)
        if attention_mask is not None:
            if attention_mask.device != x.device:
                raise ValueError("attention_mask must be on the same device as x")
            if not bool(attention_mask.bool().all()):
                raise ValueError("paged inference does not support padding masks")
        if position_ids is not None:
            expected = torch.tensor(lengths, dtype=torch.long, device=x.device)[:, None] + torch.arange(
                seq_len, device=x.device
            )
            if position_ids.shape != (batch_size, seq_len):
                raise ValueError(
                    f"position_ids must have shape {(batch_size, seq_len)}, got {tuple(position_ids.shape)}"
                )
            if position_ids.device != x.device:
                raise ValueError("position_ids must be on the same device as x")
            if not torch.equal(position_ids, expected):
                raise ValueError("position_ids must match paged cache sequence lengths")

        batch = build_ragged_batch(kv_cache, ids, (seq_len,) * batch_size, lengths)
        logits = self.run_tokens(x.reshape(-1), kv_cache, batch)
        for s in ids:
            kv_cache.advance(s, seq_len)
        return logits.view(batch_size, seq_len, -1)

    def forward_ragged(
        self,
        input_ids: torch.Tensor,
        *,
        kv_cache: PagedKVCache,
        sequence_ids: tuple[str, ...],
        query_start_loc: torch.Tensor,
        logits_rows: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Flattened variable-length prefill/decode over the paged cache.

        Returns logits for every input token (or for ``logits_rows`` only).
        """
        if input_ids.ndim != 1 or input_ids.numel() == 0:
            raise ValueError("input_ids must be a non-empty 1D tensor")
        if not isinstance(kv_cache, PagedKVCache):
            raise TypeError("kv_cache must be a PagedKVCache")
        if not sequence_ids or len(set(sequence_ids)) != len(sequence_ids):
            raise ValueError("sequence_ids must be non-empty and unique")
        if query_start_loc.ndim != 1 or query_start_loc.numel() != len(sequence_ids) + 1:
            raise ValueError("query_start_loc must have one boundary per sequence")
        if query_start_loc.device != input_ids.device:
            raise ValueError("query_start_loc must be on the input device")
        bounds = query_start_loc.tolist()
        if bounds[0] != 0 or bounds[-1] != input_ids.numel():
            raise ValueError("query_start_loc must span all input tokens")
        if any(end <= start for start, end in zip(bounds, bounds[1:])):
            raise ValueError("each ragged query must contain at least one token")
        return self._forward_packed(
            input_ids,
            kv_cache,
            tuple(sequence_ids),
            tuple(end - start for start, end in zip(bounds, bounds[1:])),
            logits_rows,
        )

    def _forward_packed(
        self,
        input_ids: torch.Tensor,
        kv_cache: PagedKVCache,
        sequence_ids: tuple[str, ...],
        query_lens: tuple[int, ...],
        logits_rows: torch.Tensor | None,
    ) -> torch.Tensor:
        context_lens = tuple(kv_cache.get_sequence_length(s) for s in sequence_ids)
        for s, ctx, q in zip(sequence_ids, context_lens, query_lens):
            if ctx + q > self.config.max_seq_len:
                raise ValueError(f"Sequence length {ctx + q} exceeds max_seq_len={self.config.max_seq_len}")
            kv_cache.ensure_capacity(s, ctx + q)
        batch = build_ragged_batch(kv_cache, sequence_ids, query_lens, context_lens)
        logits = self.run_tokens(input_ids, kv_cache, batch, logits_rows)
        for s, q in zip(sequence_ids, query_lens):
            kv_cache.advance(s, q)
        return logits
