"""Pre-norm Llama decoder block (``layers/decoder.py:23-74`` of the reference)."""

import torch
import torch.nn.functional as F
from torch import nn

from nano_infer_engine import _native
from nano_infer_engine.layers import attention as _attention
from nano_infer_engine.layers.attention import GroupedQueryAttention
from nano_infer_engine.layers.mlp import SwiGLUMLP
from nano_infer_engine.layers.rms_norm import RmsNorm


class _LeanWeights:
    """A block's parameters as ``forward_tokens_lean`` uses them: the stacked
    [q; k; v] and [gate; up] weights, the others as they are, and the norms'
    weights and eps.  ``key`` identifies the parameters it was built from."""

    __slots__ = ("key", "qkv", "qkv_sizes", "o", "gate_up", "inner", "down", "pre", "pre_eps", "post", "post_eps")


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
        self._lean: _LeanWeights | None = None  # see lean_weights

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

    def _lean_params(self):
        a, f = self.attn, self.ffn
        return ((a.q_proj, a.k_proj, a.v_proj, a.o_proj, f.gate_proj, f.up_proj, f.down_proj),
                (self.pre_norm, self.post_norm))

    def _lean_key(self, x: torch.Tensor) -> tuple:
        """What the cached lean weights depend on: x's dtype and device and,
        per projection and norm, its weight's identity, storage and version,
        whether it has a bias, and the norms' eps.  Read from the module and
        parameter dicts (every prefill-sized forward checks all blocks, and
        nn.Module attribute lookups would cost more than the check)."""
        mods = self._modules
        attn, ffn = mods["attn"]._modules, mods["ffn"]._modules
        pre, post = mods["pre_norm"], mods["post_norm"]
        key = [x.dtype, x.device, pre.eps, post.eps]
        for m in (attn["q_proj"], attn["k_proj"], attn["v_proj"], attn["o_proj"], ffn["gate_proj"], ffn["up_proj"],
                  ffn["down_proj"], pre, post):
            params = m._parameters
            w = params.get("weight")
            key += (None, 0, 0) if w is None else (id(w), w.data_ptr(), w._version)
            key.append(params.get("bias") is not None)
        return tuple(key)

    def lean_weights(self, x: torch.Tensor) -> bool:
        """Whether ``forward_tokens_lean`` takes x's rows: bias-free projections
        and weighted norms of x's dtype on x's device, in shapes the norm and
        SiLU-product kernels take.  Rebuilds the cached weights when one of
        the block's parameters was replaced or modified since."""
        key = self._lean_key(x)
        cached = self._lean
        if cached is not None and cached.key == key:
            return True
        self._lean = None
        linears, norms = self._lean_params()
        if any(m.bias is not None for m in linears) or any(n.weight is None for n in norms):
            return False
        ws = [m.weight for m in linears] + [n.weight for n in norms]
        if any(w.dtype != x.dtype or w.device != x.device for w in ws):
            return False
        hidden = self.hidden_size
        gate, up = linears[4].weight, linears[5].weight
        if (gate.shape != up.shape or any(n.weight.shape != (hidden,) for n in norms)
                or not _native.rms_norm_supported(x) or x.shape[-1] != hidden):
            return False
        inner = gate.shape[0]
        if (inner * x.element_size()) % 16:
            return False
        lean = _LeanWeights()
        lean.key = key
        lean.qkv = self.attn._stacked_qkv_weight()
        lean.qkv_sizes = tuple(m.weight.shape[0] for m in linears[:3])
        lean.o, lean.down = linears[3].weight, linears[6].weight
        lean.gate_up, lean.inner = self.ffn._stacked_gate_up_weight(), inner
        lean.pre, lean.pre_eps = norms[0].weight, float(norms[0].eps)
        lean.post, lean.post_eps = norms[1].weight, float(norms[1].eps)
        self._lean = lean
        return True

    def forward_tokens_lean(self, x, paged_cache, layer_index, batch, stream: int):
        """``forward_tokens_unsummed`` for a packed batch of many rows (a
        prefill step's), with the least host work per layer: the block's
        weights cached by ``lean_weights`` (which the caller ran for x this
        forward), torch's GEMMs, and the library's norm (residual add fused)
        and SiLU-product kernels called directly on buffers made here.  The
        same kernels and GEMMs as ``forward_tokens_unsummed`` on such a batch,
        so the same results; about 140 instead of 320 us of host time per
        block on a 544-row mixed step, below its GPU time.  x: contiguous
        (tokens, hidden) rows, or a pair of them standing for their sum."""
        w = self._lean
        a, b = x if isinstance(x, tuple) else (x, None)
        normed = torch.empty_like(a)
        if b is None:
            h = a
            _native.rms_norm_rows_into(a, None, w.pre, w.pre_eps, normed, None, stream)
        else:
            h = torch.empty_like(a)
            _native.rms_norm_rows_into(a, b, w.pre, w.pre_eps, normed, h, stream)
        attn = self.attn
        tokens = a.shape[0]
        q, k, v = F.linear(normed, w.qkv).split(w.qkv_sizes, dim=-1)
        context = _attention.attention_core(
            q.view(tokens, attn.q_head_num, attn.head_dim), k.view(tokens, attn.kv_head_num, attn.head_dim),
            v.view(tokens, attn.kv_head_num, attn.head_dim), paged_cache, layer_index, batch,
            attn.head_dim**-0.5, attn.rope,
        )
        o = F.linear(context.view(tokens, attn.hidden_size), w.o)
        h2, normed = torch.empty_like(o), torch.empty_like(o)
        _native.rms_norm_rows_into(o, h, w.post, w.post_eps, normed, h2, stream)
        act = _native.silu_mul_rows(F.linear(normed, w.gate_up), w.inner, stream)
        return F.linear(act, w.down), h2

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
