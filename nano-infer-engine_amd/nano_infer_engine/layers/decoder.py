"""Pre-norm Llama decoder block (``layers/decoder.py:23-74`` of the reference)."""

from torch import nn

from nano_infer_engine.layers.attention import GroupedQueryAttention
from nano_infer_engine.layers.mlp import SwiGLUMLP
from nano_infer_engine.layers.rms_norm import RmsNorm


class Llama3Decoder(nn.Module):
    def __init__(self, norm_eps, q_head_num, kv_head_num, hidden_size, mlp_inner_size, rope=None):
        super().__init__()
        self.q_head_num = q_head_num
        self.kv_head_num = kv_head_num
        self.hidden_size = hidden_size
        self.norm_eps = norm_eps
        self.inner_size = mlp_inner_size
        self.attn = GroupedQueryAttention(q_head_num, kv_head_num, hidden_size, rope)
        self.ffn = SwiGLUMLP(mlp_inner_size, hidden_size)
        self.pre_norm = RmsNorm(hidden_size, eps=norm_eps)
        self.post_norm = RmsNorm(hidden_size, eps=norm_eps)

    def _mlp_residual(self, attn, x):
        # h = attn + x, then ffn(post_norm(h)) + h; the add and the norm are
        # one kernel on the GPU
        h, normed = self.post_norm.forward_add(attn, x)
        return self.ffn(normed) + h

    def forward(self, x, k_cache=None, v_cache=None, cache_position=0, attention_mask=None,
                position_ids=None, *, paged_cache=None, layer_index=None, sequence_id="default",
                sequence_ids=None, paged_batch=None):
        attn = self.attn(
            self.pre_norm(x), k_cache, v_cache, cache_position, attention_mask, position_ids,
            paged_cache=paged_cache, layer_index=layer_index, sequence_id=sequence_id,
            sequence_ids=sequence_ids, paged_batch=paged_batch,
        )
        return self._mlp_residual(attn, x)

    def forward_ragged(self, x, *, paged_cache, layer_index, sequence_ids, query_start_loc,
                       context_lengths, paged_batch=None):
        attn = self.attn.forward_ragged(
            self.pre_norm(x), paged_cache=paged_cache, layer_index=layer_index,
            sequence_ids=sequence_ids, query_start_loc=query_start_loc,
            context_lengths=context_lengths, paged_batch=paged_batch,
        )
        return self._mlp_residual(attn, x)

    def forward_tokens(self, x, paged_cache, layer_index, batch):
        """Packed tokens (num_tokens, hidden) of a prebuilt ragged batch."""
        attn = self.attn.forward_tokens(self.pre_norm(x), paged_cache, layer_index, batch)
        return self._mlp_residual(attn, x)

    def forward_tokens_unsummed(self, x, paged_cache, layer_index, batch):
        """forward_tokens with the block's last residual add left to the caller.

        ``x`` is the block input, or a pair ``(a, b)`` standing for ``a + b``
        (the previous block's unsummed output): the add then happens inside
        this block's pre-attention norm (one kernel on the GPU).  Returns
        ``(ffn_out, h)``, whose sum ``ffn_out + h`` is the block's output
        (reference ``layers/decoder.py:50-51``).
        """
        a, b = x if isinstance(x, tuple) else (x, None)
        # a decode step's rows: each norm (with the residual add before it)
        # runs inside the projection GEMM that consumes it
        fused = self.attn.project_qkv_normed(a, b, self.pre_norm)
        if fused is not None:
            x, q, k, v = fused
            attn = self.attn.forward_tokens(None, paged_cache, layer_index, batch, qkv=(q, k, v))
        else:
            if b is not None:
                x, normed = self.pre_norm.forward_add(a, b)
            else:
                x, normed = a, self.pre_norm(a)
            attn = self.attn.forward_tokens(normed, paged_cache, layer_index, batch)
        out = self.ffn.forward_normed(attn, x, self.post_norm)
        if out is not None:
            return out
        h, normed = self.post_norm.forward_add(attn, x)
        return self.ffn(normed), h
