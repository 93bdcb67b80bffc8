"""The reference engine's Llama forward over a paged cache, restated in torch.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker that the
product model's end-to-end numerics are measured against, never part of the
product.

:class:`ReferenceLlama` runs ``Llama3_2.forward_ragged`` of the reference
(``src/nano_infer_engine/models/llama.py:339-394``) with the reference's
own torch ops, in the reference's order, so the rounding points are the
reference's:

* embedding lookup, then per decoder block (``layers/decoder.py:55-74``):
  ``RmsNorm`` in fp32 with one cast back (``layers/rms_norm.py:25-31``);
  separate q / k / v ``nn.Linear`` projections (``layers/attention.py:359-361``);
  RoPE at the packed positions with sin / cos of fp32 angles cast to the
  model dtype and the rotate-half products rounded one by one
  (``layers/rope.py:6-23``, ``:184-200``); per request: write the new K/V,
  gather the whole context, ``repeat_interleave`` the KV heads,
  ``q @ k^T * scale``, the causal ``masked_fill``, fp32 softmax, cast,
  ``@ v`` (``layers/attention.py:378-412``); ``o_proj``; the residual add;
  the post-attention norm; SwiGLU ``down(silu(gate(x)) * up(x))``
  (``layers/mlp.py:18-22``); the second residual add;
* the final norm and the LM head over every packed token
  (``models/llama.py:391``); the caller picks the rows it needs, as
  ``paged_prefill_chunks`` does (``generation/paged_prefill.py:150-155``).

Two departures, neither of which changes a value: the per-token gather +
``torch.stack`` of ``PagedKVCache.gather`` (``paged_cache.py:349-362``) is one
``index_select`` over the same slots (the same elements, copied), and the
right operands of the two batched products are made contiguous before the
product, which goes through ``reference_ops.batched_product`` (a bf16 bmm
over a transposed view is a known GPU-fault hazard on ROCm).

The weights are a product ``Llama3_2``'s (same parameter names as the
reference), optionally cast to another dtype: with ``dtype=torch.float32`` the
same algorithm runs in fp32 from the same bf16 weights, a high-precision
truth that both bf16 paths are measured against.  K/V live in the tensors of
the cache object passed in (``.keys`` / ``.values``, 5-D); its host methods
(``get_sequence_length``, ``ensure_capacity``, ``get_block_table``,
``advance``) do the block bookkeeping.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle.reference_ops import batched_product, rope_module_inv_freq


def rms_norm_reference(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """``RmsNorm.forward`` (``layers/rms_norm.py:25-31``)."""
    dtype = x.dtype
    h = x.float()
    h = h / torch.sqrt(torch.mean(torch.square(h), dim=-1, keepdim=True) + eps)
    if weight is not None:
        h = weight.float() * h
    return h.to(dtype)


def rope_rotate(x: torch.Tensor, sin: torch.Tensor, cos: torch.Tensor) -> torch.Tensor:
    """``_apply_rotary_emb`` (``layers/rope.py:6-23``) on packed rows (T, H, D);
    sin / cos (T, D/2) already in x's dtype."""
    first, second = x.chunk(2, dim=-1)
    sin, cos = sin[:, None, :], cos[:, None, :]
    return torch.cat((first * cos - second * sin, second * cos + first * sin), dim=-1)


class _Layer:
    __slots__ = ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "pre", "post", "eps")


class ReferenceLlama:
    """The reference's ragged forward over a product model's weights."""

    def __init__(self, model, dtype: torch.dtype | None = None, fp32_attention_products: bool = False):
        """``fp32_attention_products``: run the two attention products as fp32
        matmuls of the same operands, rounded to the model dtype at the same
        points — the same algorithm and rounding points with another
        accumulation order (a second, equally valid bf16 implementation, used
        to measure how far two such implementations drift apart)."""
        cfg = model.config
        self.config = cfg
        self.dtype = dtype or model.embed.weight.dtype
        self.fp32_products = fp32_attention_products

        def w(t: torch.Tensor) -> torch.Tensor:
            t = t.detach()
            return t if t.dtype == self.dtype else t.to(self.dtype)

        self.embed = w(model.embed.weight)
        self.lm_head = w(model.lm_head.weight)
        self.final_norm = w(model.final_rms.weight)
        self.final_eps = model.final_rms.eps
        self.layers = []
        for block in model.decoders:
            layer = _Layer()
            attn, mlp = block.attn, block.ffn
            layer.wq, layer.wk, layer.wv, layer.wo = (w(p.weight) for p in (attn.q_proj, attn.k_proj, attn.v_proj,
                                                                          attn.o_proj))
            layer.wg, layer.wu, layer.wd = (w(p.weight) for p in (mlp.gate_proj, mlp.up_proj, mlp.down_proj))
            layer.pre, layer.post = w(block.pre_norm.weight), w(block.post_norm.weight)
            layer.eps = block.pre_norm.eps
            self.layers.append(layer)
        self.q_heads, self.kv_heads, self.head_dim = cfg.q_head_num, cfg.kv_head_num, cfg.head_dim
        self.inv_freq = rope_module_inv_freq(model.rope, model.embed.weight.device)

    @torch.inference_mode()
    def forward_ragged(self, input_ids: torch.Tensor, *, kv_cache, sequence_ids: tuple[str, ...],
                       query_start_loc) -> torch.Tensor:
        """Logits of every packed token, (total_tokens, vocab), in ``self.dtype``."""
        bounds = [int(b) for b in (query_start_loc.tolist() if torch.is_tensor(query_start_loc)
                                   else query_start_loc)]
        query_lens = [b - a for a, b in zip(bounds, bounds[1:])]
        context = [kv_cache.get_sequence_length(s) for s in sequence_ids]
        for s, ctx, n in zip(sequence_ids, context, query_lens):
            kv_cache.ensure_capacity(s, ctx + n)
        device = input_ids.device
        bs = kv_cache.block_size
        # per request: the flat slots of positions 0 .. ctx + n - 1 (one copy
        # for the whole forward), and the new tokens' positions
        slots, positions = [], []
        for s, ctx, n in zip(sequence_ids, context, query_lens):
            table = np.asarray(kv_cache.get_block_table(s), dtype=np.int64)
            pos = np.arange(ctx + n, dtype=np.int64)
            slots.append(table[pos // bs] * bs + pos % bs)
            positions.append(pos[ctx:])
        sizes = [len(x) for x in slots]
        flat = torch.from_numpy(np.concatenate(slots)).to(device)
        slot_rows = list(flat.split(sizes))
        pos_t = torch.from_numpy(np.concatenate(positions)).to(device)
        angles = pos_t.to(torch.float32)[:, None] * self.inv_freq
        sin, cos = torch.sin(angles).to(self.dtype), torch.cos(angles).to(self.dtype)

        x = F.embedding(input_ids, self.embed)
        for index, layer in enumerate(self.layers):
            h = self._attention(rms_norm_reference(x, layer.pre, layer.eps), layer, kv_cache, index, bounds,
                                context, slot_rows, sin, cos) + x
            m = rms_norm_reference(h, layer.post, layer.eps)
            x = F.linear(F.silu(F.linear(m, layer.wg)) * F.linear(m, layer.wu), layer.wd) + h
        logits = F.linear(rms_norm_reference(x, self.final_norm, self.final_eps), self.lm_head)
        for s, n in zip(sequence_ids, query_lens):
            kv_cache.advance(s, n)
        return logits

    def _attention(self, x, layer, cache, index, bounds, context, slot_rows, sin, cos) -> torch.Tensor:
        tokens = x.shape[0]
        hq, hkv, d = self.q_heads, self.kv_heads, self.head_dim
        group = hq // hkv
        q = rope_rotate(F.linear(x, layer.wq).view(tokens, hq, d), sin, cos)
        k = rope_rotate(F.linear(x, layer.wk).view(tokens, hkv, d), sin, cos)
        v = F.linear(x, layer.wv).view(tokens, hkv, d)
        keys = cache.keys[index].view(-1, hkv, d)
        values = cache.values[index].view(-1, hkv, d)
        scale = d**-0.5
        out = []
        for r, (start, end) in enumerate(zip(bounds, bounds[1:])):
            ctx, total = context[r], context[r] + end - start
            rows = slot_rows[r]
            keys[rows[ctx:]] = k[start:end]
            values[rows[ctx:]] = v[start:end]
            ks = keys.index_select(0, rows).repeat_interleave(group, dim=1)
            vs = values.index_select(0, rows).repeat_interleave(group, dim=1)
            query = q[start:end].transpose(0, 1)
            keys_t = ks.transpose(0, 1).transpose(-1, -2).contiguous()
            if self.fp32_products:
                scores = batched_product(query.float(), keys_t.float()).to(query.dtype) * scale
            else:
                scores = batched_product(query, keys_t) * scale
            q_pos = torch.arange(ctx, total, device=x.device)[:, None]
            k_pos = torch.arange(total, device=x.device)[None, :]
            scores = scores.masked_fill(k_pos > q_pos, float("-inf"))
            probs = torch.softmax(scores, dim=-1, dtype=torch.float32)
            values_t = vs.transpose(0, 1).contiguous()
            if self.fp32_products:
                context_rows = batched_product(probs.to(vs.dtype).float(), values_t.float()).to(vs.dtype)
            else:
                context_rows = batched_product(probs.to(vs.dtype), values_t)
            out.append(context_rows.transpose(0, 1).reshape(end - start, hq * d))
        return F.linear(torch.cat(out, dim=0), layer.wo)
