"""HIP-graph replay of the all-decode step (one new token per request).

The reference runs every decode iteration eagerly from Python and lists
graph capture of stable decode shapes as future work
(``docs/development-roadmap.md:89``, ``:190``).  Here the whole step of a
:class:`~nano_infer_engine.models.llama.Llama3_2` — embedding, every layer
(projections, fused RoPE + KV append, paged decode attention, MLP), final
norm, LM head and the greedy argmax — is captured once per (batch size,
length bucket) and replayed:

* the step's inputs live in one static device buffer: slot mapping,
  positions, ``cu_seqlens`` and token IDs (int64), block tables (width =
  bucket / block_size) and context and sequence lengths (int32); its pinned
  host staging persists with the capture, its tables updated in place
  (:class:`~nano_infer_engine.paged_batch.TableMirror`: only a sequence's new
  blocks, or a row that changed hands), and one host-to-device copy
  refreshes the device side per step (the token IDs included when the
  caller has them on the host, as the scheduler does after reading the last
  step's tokens);
* the decode launch inside the graph is sized for the bucket
  (:func:`~nano_infer_engine.paged_batch.decode_plan_bound`) and takes its
  work items from the exact plan of the step's lengths, which travels in
  the same buffer (``_native.write_decode_plan``), so a replay computes the
  same values as the eager step, planned from the same host lengths;
* the graph ends with :func:`~nano_infer_engine._native.argmax_rows`, so the
  next token IDs are on the device when the replay finishes.

Steps that carry prefill chunks, batches larger than ``max_batch_size`` and
sequences past ``max_graph_len`` run eagerly.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass

import numpy as np
import torch

from nano_infer_engine import _native
from nano_infer_engine.paged_batch import RaggedBatch, TableMirror, decode_plan_bound
from nano_infer_engine.paged_cache import PagedKVCache


@dataclass
class _CapturedStep:
    graph: torch.cuda.CUDAGraph
    batch: RaggedBatch
    meta: torch.Tensor  # device bytes: ``longs``, ``ids``, ``ints``, then the decode plan
    ids: torch.Tensor  # (B,) int64 input token IDs (a view of ``meta``)
    meta_host: torch.Tensor  # pinned staging of ``meta``
    ints_np: np.ndarray  # staging views: tables (B*W), context lens (B), sequence lens (B)
    longs_np: np.ndarray  # slots (B), positions (B), cu_seqlens (B + 1)
    ids_np: np.ndarray  # token IDs (B)
    plan_at: int  # byte offset of the decode plan in ``meta``
    width: int
    copied: torch.cuda.Event  # recorded after the staging copies of the last step
    logits: torch.Tensor  # (B, vocab) output of the last replay (its own buffer, outside the graph pool)
    next_ids: torch.Tensor  # (B,) int64 argmax of ``logits``
    mirror: TableMirror  # the staged tables, updated in place from step to step


class DecodeGraphRunner:
    """Captures and replays the decode step of ``model`` over ``cache``."""

    def __init__(self, model, cache: PagedKVCache, max_batch_size: int, max_graph_len: int = 32768,
                 max_graphs: int = 64):
        if cache.keys.device.type != "cuda":
            raise RuntimeError("decode graphs need the cache on a ROCm GPU")
        if max_graphs < 1:
            raise ValueError("max_graphs must be positive")
        self.model = model
        self.cache = cache
        self.max_batch_size = max_batch_size
        self.max_graph_len = max_graph_len
        self.max_graphs = max_graphs
        self.device = cache.keys.device
        # captures run on a side stream of default priority
        self._stream = torch.cuda.Stream(self.device)
        # Every capture allocates from one shared memory pool: the steps never
        # run concurrently (one stream), so their activations can share
        # memory, and each step's outputs (logits, next IDs) stay referenced by
        # its _CapturedStep, so no other capture is handed them.  A KV pool
        # sized to most of HBM then leaves room for one set of activations
        # plus a B x vocab logits buffer per graph, not a private pool each.
        self._pool = torch.cuda.graph_pool_handle()
        # least recently replayed first; at most max_graphs are kept
        self._steps: OrderedDict[tuple[int, int], _CapturedStep] = OrderedDict()
        self.captures = 0
        self.replays = 0
        self.evictions = 0

    def supports(self, batch_size: int, max_seq_len: int) -> bool:
        return 0 < batch_size <= self.max_batch_size and decode_plan_bound(max_seq_len) <= self.max_graph_len

    # ---------------------------------------------------------------- capture
    def _capture(self, batch_size: int, bound: int) -> _CapturedStep:
        cache, model = self.cache, self.model
        b, width = batch_size, -(-bound // cache.block_size)
        # one buffer, so a step's inputs are one copy: int64 slots, positions,
        # cu_seqlens and token IDs first (8-byte aligned), then the int32s
        n_long, n_int = 4 * b + 1, b * width + 2 * b
        plan_at = -(-(8 * n_long + 4 * n_int) // 16) * 16
        meta = torch.zeros(plan_at + _native.decode_plan_bytes(), dtype=torch.uint8, device=self.device)
        longs = meta[: 8 * (3 * b + 1)].view(torch.int64)
        ids = meta[8 * (3 * b + 1) : 8 * n_long].view(torch.int64)
        ints = meta[8 * n_long : 8 * n_long + 4 * n_int].view(torch.int32)
        # capture-time contents: length-1 sequences at position 0 whose
        # table entries lie outside the pool and whose slots are -1, so the
        # K/V writes of the warm-up and capture runs are skipped (the fused
        # decode derives its slot from the table; reads clamp into the pool)
        ints[: b * width] = cache.keys.shape[1]
        ints[b * width :] = 1
        ints[b * width : b * width + b] = 0
        longs[:b] = -1
        longs[2 * b :] = torch.arange(b + 1, device=self.device)
        batch = RaggedBatch(
            sequence_ids=tuple(f"graph-row-{i}" for i in range(b)),
            query_lens=(1,) * b,
            context_lens=(bound - 1,) * b,  # sizes the RoPE tables for the bucket
            num_tokens=b,
            block_tables=ints[: b * width].view(b, width),
            context_lens_t=ints[b * width : b * width + b],
            seq_lens_t=ints[b * width + b :],
            cu_seqlens=longs[2 * b :],
            slot_mapping=longs[:b],
            positions=longs[b : 2 * b],
            decode_from=0,
            decode_bound=bound,
            decode_plan=meta[plan_at:],  # zeros at capture: planned from the bounds
        )
        next_ids = torch.zeros(b, dtype=torch.int64, device=self.device)
        stream = self._stream
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream), torch.inference_mode():
            # eager warm-up on the capture stream: builds the launches (which
            # remember this stream), their workspaces and the GEMM plans
            logits = model.run_tokens(ids, cache, batch)
            # the step's logits are copied into a buffer of its own, outside
            # the shared graph pool, so replaying another capture (whose
            # activations may reuse this capture's pool blocks) leaves them
            # intact until this capture replays again
            out_logits = torch.empty_like(logits)
            out_logits.copy_(logits)
            _native.argmax_rows(out_logits, out=next_ids)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream, pool=self._pool):
                logits = model.run_tokens(ids, cache, batch)
                out_logits.copy_(logits)
                _native.argmax_rows(out_logits, out=next_ids)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        self.captures += 1
        meta_host = torch.empty(meta.shape, dtype=torch.uint8, pin_memory=True)
        staged = meta_host.numpy()
        return _CapturedStep(
            graph=graph,
            batch=batch,
            meta=meta,
            ids=ids,
            meta_host=meta_host,
            ints_np=staged[8 * n_long : 8 * n_long + 4 * n_int].view(np.int32),
            longs_np=staged[: 8 * (3 * b + 1)].view(np.int64),
            ids_np=staged[8 * (3 * b + 1) : 8 * n_long].view(np.int64),
            plan_at=plan_at,
            width=width,
            copied=torch.cuda.Event(),
            logits=out_logits,
            next_ids=next_ids,
            mirror=TableMirror(),
        )

    # ------------------------------------------------------------------ step
    @torch.inference_mode()
    def step(self, token_ids: torch.Tensor | None, sequence_ids: tuple[str, ...],
             host_ids: list[int] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Append one token per sequence and run the model: returns (logits (B, vocab), next IDs (B,)).

        Both are the capture's own output buffers (outside the graph memory
        pool the captures share), valid until the next call with the same
        batch size and bucket; replays of other captures leave them alone.  Validation and cache bookkeeping follow
        the eager path (``Llama3_2._forward_packed``).  ``host_ids``: the
        token IDs as a host list, in place of ``token_ids`` (None); they then
        travel with the step's metadata copy instead of in a device copy.
        ``sequence_ids`` must be the scheduler's checked IDs.
        """
        cache, config = self.cache, self.model.config
        b = len(sequence_ids)
        given = len(host_ids) if host_ids is not None else (-1 if token_ids is None else token_ids.numel())
        if given != b:
            raise ValueError("one token per sequence is required")
        context = cache._lengths(sequence_ids)
        for ctx in context:
            if ctx + 1 > config.max_seq_len:
                raise ValueError(f"Sequence length {ctx + 1} exceeds max_seq_len={config.max_seq_len}")
        rows = cache._reserve_next(sequence_ids, context)
        bound = decode_plan_bound(max(context) + 1)
        if not self.supports(b, max(context) + 1):
            raise ValueError("batch size or sequence length outside the captured range")
        key = (b, bound)
        step = self._steps.get(key)
        if step is None:
            if len(self._steps) >= self.max_graphs:
                # drop the least recently replayed capture (its logits stay
                # alive while a request still holds a view of them)
                _, old = self._steps.popitem(last=False)
                old.copied.synchronize()
                del old
                self.evictions += 1
            step = self._capture(b, bound)
            self._steps[key] = step
        else:
            self._steps.move_to_end(key)

        # host metadata into the pinned staging buffers (once the previous
        # step's copies out of them have run), then one copy each
        step.copied.synchronize()
        bs, width = cache.block_size, step.width
        ints, longs = step.ints_np, step.longs_np
        tables = ints[: b * width].reshape(b, width)
        # only the table entries that changed since this capture's last
        # replay are rewritten (a new block per sequence every block_size steps)
        step.mirror.fill(tables, rows)
        ctx = np.asarray(context, dtype=np.int64)
        ints[b * width : b * width + b] = ctx
        ints[b * width + b :] = ctx + 1
        longs[:b] = tables[np.arange(b), ctx // bs].astype(np.int64) * bs + ctx % bs
        longs[b : 2 * b] = ctx
        longs[2 * b :] = np.arange(b + 1)
        lens = ints[b * width + b :]  # context + 1
        keys = cache.keys
        _native.write_decode_plan(step.meta_host.data_ptr() + step.plan_at, step.meta_host.numel() - step.plan_at,
                                  keys.dtype, config.q_head_num, keys.shape[3], keys.shape[4], bs, lens,
                                  int(ctx.max()) + 1, int(ctx.sum()) + b)
        if host_ids is not None:
            step.ids_np[:] = host_ids
        step.meta.copy_(step.meta_host, non_blocking=True)
        step.copied.record()
        if host_ids is None:
            step.ids.copy_(token_ids.reshape(-1))
        step.graph.replay()
        self.replays += 1
        cache._advance_reserved(sequence_ids)
        return step.logits, step.next_ids
