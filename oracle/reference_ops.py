"""Loop-for-loop torch restatement of the reference hot path.  Test infrastructure only.

Each function follows the cited lines of ito-integral/nano-infer-engine
(``src/nano_infer_engine/...``), using the same torch ops in the same order
so the rounding points match: bf16 q.k via einsum/matmul, ``* scale`` in the
storage dtype, fp32 softmax, probabilities cast back to the storage dtype,
P.V via einsum/matmul.  Works on any device (CPU for the baseline and the
CPU tests, the GPU for the reference-PyTorch-path comparison).
"""

from __future__ import annotations

import math

import torch


def batched_product(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b`` for the oracle's batched products, refusing the one form known
    to be unsafe on ROCm GPUs: a bf16 batched product (``torch.bmm`` and what
    ``matmul`` / ``einsum`` lower to) whose right operand is a transposed,
    non-contiguous view can fault the device.  Every caller makes its right
    operand contiguous first; this check keeps it that way (ValueError)."""
    if b.is_cuda and b.dtype == torch.bfloat16 and b.dim() >= 3 and not b.is_contiguous():
        raise ValueError("a bf16 batched product on the GPU needs a contiguous right operand")
    return a @ b


def paged_attention_reference(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: tuple[int, ...],
    sequence_length: int,
    layer_index: int,
) -> torch.Tensor:
    """Decode attention by a loop over logical blocks.

    Follows ``layers/paged_attention.py:68-114``: slice the valid rows of
    each physical block, expand KV heads with repeat_interleave, score with
    einsum("hd,thd->ht") times head_dim**-0.5, concatenate in logical order,
    fp32 softmax cast back to the input dtype, einsum("ht,thd->hd").
    """
    _, _, block_size, kv_heads, head_dim = key_cache.shape
    q_heads = query.shape[0]
    group = q_heads // kv_heads
    blocks = -(-sequence_length // block_size)
    scores, values = [], []
    for logical, physical in enumerate(block_table[:blocks]):
        valid = min(block_size, sequence_length - logical * block_size)
        k_rows = key_cache[layer_index, physical, :valid].repeat_interleave(group, dim=1)
        v_rows = value_cache[layer_index, physical, :valid].repeat_interleave(group, dim=1)
        scores.append(torch.einsum("hd,thd->ht", query, k_rows) * (head_dim**-0.5))
        values.append(v_rows)
    weights = torch.softmax(torch.cat(scores, dim=-1), dim=-1, dtype=torch.float32).to(query.dtype)
    return torch.einsum("ht,thd->hd", weights, torch.cat(values, dim=0))


def batched_paged_attention_reference(query, key_cache, value_cache, block_tables, sequence_lengths, layer_index):
    """Per-sequence loop + stack (``layers/paged_attention.py:164-176``)."""
    return torch.stack(
        [
            paged_attention_reference(query[b], key_cache, value_cache, block_tables[b], sequence_lengths[b], layer_index)
            for b in range(query.shape[0])
        ],
        dim=0,
    )


def paged_attention_reference_matmul(query, key_cache, value_cache, block_table, sequence_length, layer_index):
    """:func:`paged_attention_reference` with each ``einsum`` written as a
    batched ``matmul`` over contiguous operands (head-major), for timing the
    reference's per-block loop on a ROCm GPU, where a bf16 batched product
    over a transposed operand (what einsum forms inside) is a known fault
    hazard (:func:`batched_product`).  The
    loop, the repeat_interleave, the scale, the fp32 softmax and the casts
    are the reference's (``layers/paged_attention.py:82-114``)."""
    _, _, block_size, kv_heads, head_dim = key_cache.shape
    group = query.shape[0] // kv_heads
    blocks = -(-sequence_length // block_size)
    scores, values = [], []
    for logical, physical in enumerate(block_table[:blocks]):
        valid = min(block_size, sequence_length - logical * block_size)
        k_rows = key_cache[layer_index, physical, :valid].repeat_interleave(group, dim=1)
        v_rows = value_cache[layer_index, physical, :valid].repeat_interleave(group, dim=1)
        k_t = k_rows.permute(1, 2, 0).contiguous()  # (Hq, D, valid)
        scores.append(batched_product(query[:, None, :], k_t)[:, 0, :] * (head_dim**-0.5))
        values.append(v_rows)
    weights = torch.softmax(torch.cat(scores, dim=-1), dim=-1, dtype=torch.float32).to(query.dtype)
    v_all = torch.cat(values, dim=0).transpose(0, 1).contiguous()  # (Hq, S, D)
    return batched_product(weights[:, None, :], v_all)[:, 0, :]


def batched_paged_attention_reference_matmul(query, key_cache, value_cache, block_tables, sequence_lengths,
                                             layer_index):
    """Per-sequence loop + stack of :func:`paged_attention_reference_matmul`."""
    return torch.stack(
        [
            paged_attention_reference_matmul(query[b], key_cache, value_cache, block_tables[b], sequence_lengths[b],
                                             layer_index)
            for b in range(query.shape[0])
        ],
        dim=0,
    )


def write_tokens(keys, values, layer_index, table, block_size, start_position, new_keys, new_values) -> None:
    """Per-token scatter into the pool (``paged_cache.py:306-322``)."""
    for t in range(new_keys.shape[0]):
        logical, offset = divmod(start_position + t, block_size)
        physical = table[logical]
        keys[layer_index, physical, offset].copy_(new_keys[t])
        values[layer_index, physical, offset].copy_(new_values[t])


def gather_tokens(keys, values, layer_index, table, block_size, token_count):
    """Per-token gather + stack in logical order (``paged_cache.py:349-362``)."""
    k_rows, v_rows = [], []
    for p in range(token_count):
        logical, offset = divmod(p, block_size)
        physical = table[logical]
        k_rows.append(keys[layer_index, physical, offset])
        v_rows.append(values[layer_index, physical, offset])
    return torch.stack(k_rows), torch.stack(v_rows)


def ragged_attention_reference(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    layer_index: int,
    tables,
    context_lens,
    query_lens,
    scale: float,
) -> torch.Tensor:
    """Flattened varlen attention, one request at a time.

    Follows ``layers/attention.py:378-412``: write the request's new K/V,
    gather its whole context, repeat_interleave KV heads, ``q @ k^T * scale``,
    mask key_pos > query_pos with -inf, fp32 softmax cast to the value
    dtype, ``@ v``; contexts concatenated in request order.
    q (T, Hq, D); k, v (T, Hkv, D) -> (T, Hq, D).
    """
    block_size = keys.shape[2]
    group = q.shape[1] // k.shape[1]
    outputs = []
    start = 0
    for table, ctx, n in zip(tables, context_lens, query_lens):
        end = start + n
        write_tokens(keys, values, layer_index, table, block_size, ctx, k[start:end], v[start:end])
        total = ctx + n
        ks, vs = gather_tokens(keys, values, layer_index, table, block_size, total)
        # right operands of the batched products made contiguous (see
        # batched_product)
        ks = ks.repeat_interleave(group, dim=1).transpose(0, 1)
        vs = vs.repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
        query = q[start:end].transpose(0, 1)
        scores = batched_product(query, ks.transpose(-1, -2).contiguous()) * scale
        q_pos = torch.arange(ctx, total, device=q.device)[:, None]
        k_pos = torch.arange(total, device=q.device)[None, :]
        scores = scores.masked_fill(k_pos > q_pos, float("-inf"))
        probs = torch.softmax(scores, dim=-1, dtype=torch.float32)
        outputs.append(batched_product(probs.to(vs.dtype), vs).transpose(0, 1))
        start = end
    return torch.cat(outputs, dim=0)


def ragged_attention_reference_vectorized(q, k, v, keys, values, layer_index, tables, context_lens, query_lens,
                                          scale: float) -> torch.Tensor:
    """:func:`ragged_attention_reference` with the per-token write and gather
    each done as one indexed copy over the request's flat slots (the same
    elements, so the same values), for timing the reference's per-request
    loop on a GPU without its per-token launches."""
    block_size, hkv, d = keys.shape[2], keys.shape[3], keys.shape[4]
    group = q.shape[1] // k.shape[1]
    flat_k = keys[layer_index].view(-1, hkv, d)
    flat_v = values[layer_index].view(-1, hkv, d)
    outputs = []
    start = 0
    for table, ctx, n in zip(tables, context_lens, query_lens):
        end, total = start + n, ctx + n
        pos = torch.arange(total, device=q.device)
        slots = torch.as_tensor(list(table), device=q.device)[pos // block_size] * block_size + pos % block_size
        flat_k[slots[ctx:]] = k[start:end]
        flat_v[slots[ctx:]] = v[start:end]
        ks = flat_k.index_select(0, slots).repeat_interleave(group, dim=1).transpose(0, 1)
        vs = flat_v.index_select(0, slots).repeat_interleave(group, dim=1).transpose(0, 1).contiguous()
        scores = batched_product(q[start:end].transpose(0, 1), ks.transpose(-1, -2).contiguous()) * scale
        scores = scores.masked_fill(pos[None, :] > pos[ctx:, None], float("-inf"))
        probs = torch.softmax(scores, dim=-1, dtype=torch.float32)
        outputs.append(batched_product(probs.to(vs.dtype), vs).transpose(0, 1))
        start = end
    return torch.cat(outputs, dim=0)


def rope_inv_freq(dim: int, theta_base: float, scaling: dict | None = None, device=None) -> torch.Tensor:
    """Inverse frequencies of the reference RoPE.

    Plain: ``1 / theta ** (arange(0, dim, 2) / dim)`` (``layers/rope.py:33-35``).
    With ``scaling`` (keys factor, low_freq_factor, high_freq_factor,
    original_max_position_embeddings) the llama3 banded rescale of
    ``layers/rope.py:99-147``: wavelengths above old_ctx/low are divided by the
    factor, those below old_ctx/high kept, the band between interpolated.
    """
    i = torch.arange(0, dim, 2, dtype=torch.float32, device=device)
    inv_freq = 1 / theta_base ** (i / dim)
    if scaling is None:
        return inv_freq
    wavelen = 2 * math.pi / inv_freq
    old_ctx = scaling["original_max_position_embeddings"]
    low_freq_wavelen = old_ctx / scaling["low_freq_factor"]
    high_freq_wavelen = old_ctx / scaling["high_freq_factor"]
    scaled_inv_freq = inv_freq / scaling["factor"]
    smooth_factor = (old_ctx / wavelen - scaling["low_freq_factor"]) / (
        scaling["high_freq_factor"] - scaling["low_freq_factor"]
    )
    smooth_inv_freq = (1 - smooth_factor) * scaled_inv_freq + smooth_factor * inv_freq
    is_low_freq = wavelen > low_freq_wavelen
    is_high_freq = wavelen < high_freq_wavelen
    is_medium_freq = ~(is_low_freq | is_high_freq)
    inv_freq = torch.where(is_low_freq, scaled_inv_freq, inv_freq)
    return torch.where(is_medium_freq, smooth_inv_freq, inv_freq)


def rope_reference(x: torch.Tensor, positions: torch.Tensor, inv_freq: torch.Tensor) -> torch.Tensor:
    """RoPE of packed rows x (T, H, D) at int64 ``positions`` (T,).

    Follows the position_ids branches of ``layers/rope.py:59-75`` and
    ``:184-200`` (fp32
    angles ``position * inv_freq``, sin/cos cast to x's dtype) and
    ``_apply_rotary_emb`` (``layers/rope.py:6-23``): halves by ``chunk``,
    ``(x1*cos - x2*sin, x2*cos + x1*sin)`` concatenated.
    """
    angles = positions.to(device=x.device, dtype=torch.float32)[:, None] * inv_freq
    sin = torch.sin(angles).to(x.dtype)[:, None, :]
    cos = torch.cos(angles).to(x.dtype)[:, None, :]
    x_first, x_second = x.chunk(2, dim=-1)
    return torch.cat((x_first * cos - x_second * sin, x_second * cos + x_first * sin), dim=-1)


def rope_module_inv_freq(rope, device) -> torch.Tensor:
    """:func:`rope_inv_freq` for the hyperparameters of a product RoPE module."""
    scaling = None
    if hasattr(rope, "scaling_factor"):
        scaling = {
            "factor": rope.scaling_factor,
            "low_freq_factor": rope.low_freq_factor,
            "high_freq_factor": rope.high_freq_factor,
            "original_max_position_embeddings": rope.original_max_position_embeddings,
        }
    return rope_inv_freq(rope.dim, rope.theta_base, scaling, device)


def attention_core_like_product(q, k, v, cache, layer_index, batch, scale, rope):
    """Same contract as the product's per-layer attention core (q, k not yet
    rotated): :func:`rope_reference` on q and k, then
    :func:`ragged_attention_reference` on the cache's storage tensors.

    Used to run the product model with the reference algorithm swapped in
    (the "reference PyTorch path" of the end-to-end comparison).
    """
    inv_freq = rope_module_inv_freq(rope, q.device)
    q = rope_reference(q, batch.positions, inv_freq)
    k = rope_reference(k, batch.positions, inv_freq)
    tables = [cache.get_block_table(s) for s in batch.sequence_ids]
    return ragged_attention_reference(
        q, k, v, cache.keys, cache.values, layer_index, tables, batch.context_lens, batch.query_lens, scale
    )
