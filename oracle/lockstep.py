"""Step-by-step comparison of a product serving run with the reference algorithm.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

:func:`run_lockstep` serves prompts through the product's
``ContinuousBatchingScheduler`` exactly as shipped (chunked prefill, decode
HIP graphs, the library GEMMs) and, after every scheduler step, replays that
step's forward — the same sequence IDs, query lengths and input token IDs,
read from ``scheduler.last_plan`` — on :class:`oracle.reference_model.ReferenceLlama`
in bf16 (the reference path) and in fp32 (a higher-precision truth from the
same weights), each over a cache of its own.  The reference models are
teacher-forced: they consume the product's tokens, so every compared row
has an identical token history, and the first row whose argmax differs is
the step where a free-running reference path would first diverge (the batch
composition depends only on prompt lengths, so it is the same either way).

For every logits row the scheduler samples from (every decode row, and the
row of a prompt's last piece) it records the three argmaxes, the top-2
margins and the max-abs logit differences between the paths.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from oracle.reference_model import ReferenceLlama


@dataclass
class RowRecord:
    sequence_id: str
    token_index: int  # which generated token this row's argmax becomes (1-based)
    product: int
    reference: int
    truth: int
    reference_margin: float  # top-1 minus top-2 logit of the reference row
    product_margin: float
    truth_margin: float
    err_product_reference: float  # max |product - reference| over the row
    err_product_truth: float
    err_reference_truth: float
    # truth's logit gap between the reference's and the product's choices
    # (truth[reference] - truth[product]; 0 when they agree)
    truth_gap: float
    # the reference variant (same algorithm, fp32 attention products): its
    # argmax and max |variant - reference| (-1 when it was not run)
    variant: int = -1
    err_variant_reference: float = -1.0


@dataclass
class LockstepReport:
    rows: list[RowRecord] = field(default_factory=list)
    steps: int = 0
    product_seconds: float = 0.0
    reference_seconds: float = 0.0  # the bf16 reference path's forwards
    sequences: dict[str, torch.Tensor] = field(default_factory=dict)  # the product's tokens, per request

    def first_divergence(self, other: str = "product") -> dict[str, RowRecord | None]:
        """Per request, its first row whose ``other`` ("product" or "variant")
        and reference argmaxes differ."""
        out: dict[str, RowRecord | None] = {}
        for row in sorted(self.rows, key=lambda r: r.token_index):
            out.setdefault(row.sequence_id, None)
            if out[row.sequence_id] is None and getattr(row, other) != row.reference:
                out[row.sequence_id] = row
        return out

    def summary(self) -> dict:
        rows = self.rows
        n = len(rows)
        diverged = self.first_divergence()
        flips = [r for r in rows if r.product != r.reference]

        def frac(pred):
            return round(sum(1 for r in rows if pred(r)) / max(n, 1), 5)

        def q(values, p):
            values = sorted(values)
            return round(values[min(len(values) - 1, int(p * len(values)))], 5) if values else None

        per_request = {}
        for sid, row in diverged.items():
            per_request[sid] = None if row is None else {
                "token": row.token_index, "reference_margin": round(row.reference_margin, 5),
                "product_margin": round(row.product_margin, 5),
                "err_product_reference": round(row.err_product_reference, 5),
                "truth_gap": round(row.truth_gap, 5), "truth_agrees_with": (
                    "product" if row.truth == row.product else "reference" if row.truth == row.reference else "neither"),
            }
        return {
            "requests": len(diverged),
            "sampled_rows": n,
            "steps": self.steps,
            "identical_requests": sum(1 for v in diverged.values() if v is None),
            "top1_agreement_product_reference": frac(lambda r: r.product == r.reference),
            "top1_agreement_product_truth": frac(lambda r: r.product == r.truth),
            "top1_agreement_reference_truth": frac(lambda r: r.reference == r.truth),
            "err_product_reference": {"median": q([r.err_product_reference for r in rows], 0.5),
                                      "p99": q([r.err_product_reference for r in rows], 0.99),
                                      "max": q([r.err_product_reference for r in rows], 1.0)},
            "err_product_truth": {"median": q([r.err_product_truth for r in rows], 0.5),
                                  "p99": q([r.err_product_truth for r in rows], 0.99)},
            "err_reference_truth": {"median": q([r.err_reference_truth for r in rows], 0.5),
                                    "p99": q([r.err_reference_truth for r in rows], 0.99)},
            "flips": len(flips),
            "max_reference_margin_at_flip": q([r.reference_margin for r in flips], 1.0),
            "max_truth_gap_at_flip": q([abs(r.truth_gap) for r in flips], 1.0),
            "first_divergence": per_request,
            **self._variant_summary(frac, q),
        }

    def _variant_summary(self, frac, q) -> dict:
        if not self.rows or self.rows[0].variant < 0:
            return {}
        firsts = self.first_divergence("variant")
        return {"variant": {
            "top1_agreement_variant_reference": frac(lambda r: r.variant == r.reference),
            "top1_agreement_variant_truth": frac(lambda r: r.variant == r.truth),
            "err_variant_reference": {"median": q([r.err_variant_reference for r in self.rows], 0.5),
                                      "p99": q([r.err_variant_reference for r in self.rows], 0.99)},
            "identical_requests": sum(1 for v in firsts.values() if v is None),
            "first_divergence_tokens": sorted(v.token_index for v in firsts.values() if v is not None),
        }}


def _top2(rows: torch.Tensor):
    f = rows.float()
    top1 = f.argmax(dim=-1)
    vals = f.topk(2, dim=-1).values
    return f, top1, vals[:, 0] - vals[:, 1]


def run_lockstep(model, prompts, cache_factory, *, max_new_tokens: int, max_batch_size: int, chunk: int,
                 budget: int, decode_graphs: bool = True, truth: bool = True, variant: bool = False) -> LockstepReport:
    """Serve ``prompts`` with the product and replay every step on the reference paths.

    ``cache_factory(dtype)`` returns an empty paged cache of the serving
    geometry in that dtype (one for the product, one per reference path).
    ``truth``: also the fp32 restatement; ``variant``: also the bf16
    restatement with fp32 attention products (the same algorithm with another
    accumulation order), whose distance from the reference path is what two
    valid bf16 implementations of it drift apart by.
    """
    from nano_infer_engine.generation import ContinuousBatchingScheduler, GenerationConfig

    device = model.embed.weight.device
    config = GenerationConfig(max_new_tokens=max_new_tokens, eos_token_id=None, prefill_chunk_size=chunk,
                              max_prefill_tokens_per_step=budget)
    cache = cache_factory(model.embed.weight.dtype)
    sched = ContinuousBatchingScheduler(model, config, cache, max_batch_size, decode_graphs=decode_graphs)
    requests = [sched.add_request(f"request-{i}", p) for i, p in enumerate(prompts)]
    dtype = model.embed.weight.dtype
    paths = {"reference": (ReferenceLlama(model), cache_factory(dtype))}
    if truth:
        paths["truth"] = (ReferenceLlama(model, torch.float32), cache_factory(torch.float32))
    if variant:
        paths["variant"] = (ReferenceLlama(model, fp32_attention_products=True), cache_factory(dtype))
    report = LockstepReport()
    while sched.has_work:
        before = sched.last_plan
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        sched.step()
        torch.cuda.synchronize(device)
        report.product_seconds += time.perf_counter() - t0
        report.steps += 1
        if report.steps % 50 == 0:
            print(f"lockstep: {report.steps} steps, {len(report.rows)} sampled rows", flush=True)
        plan = sched.last_plan
        for ref_model, ref_cache in paths.values():  # mirror the product's releases
            for sid in list(ref_cache._block_tables):
                if not cache.has_sequence(sid):
                    ref_cache.release(sid)
        if plan is None or plan is before:
            continue
        # rows the scheduler will sample: decode rows, and a prompt's last piece
        sampled = [(row, r) for row, (r, _, stop) in enumerate(plan.pieces) if stop == r.prompt.shape[1]]
        sampled += [(len(plan.pieces) + i, r) for i, r in enumerate(plan.decode)]
        ids = plan.input_ids()
        bounds = [0]
        for n in plan.query_lens:
            bounds.append(bounds[-1] + n)
        last = torch.tensor(bounds[1:], device=device) - 1
        outs = {}
        for name, (ref_model, ref_cache) in paths.items():
            torch.cuda.synchronize(device)
            t0 = time.perf_counter()
            logits = ref_model.forward_ragged(ids, kv_cache=ref_cache, sequence_ids=plan.sequence_ids,
                                              query_start_loc=bounds)[last]
            torch.cuda.synchronize(device)
            if name == "reference":
                report.reference_seconds += time.perf_counter() - t0
            outs[name] = logits
        if not sampled:
            continue
        rows_idx = torch.tensor([row for row, _ in sampled], device=device)
        prod = torch.stack([r.last_logits for _, r in sampled])
        p, p1, pm = _top2(prod)
        r_, r1, rm = _top2(outs["reference"][rows_idx])
        if truth:
            t, t1, tm = _top2(outs["truth"][rows_idx])
            e_pt = (p - t).abs().amax(-1)
            e_rt = (r_ - t).abs().amax(-1)
            gap = t.gather(1, r1[:, None])[:, 0] - t.gather(1, p1[:, None])[:, 0]
        else:
            t1, tm, e_pt, e_rt, gap = p1, pm, pm * 0, pm * 0, pm * 0
        e_pr = (p - r_).abs().amax(-1)
        if variant:
            v, v1, _ = _top2(outs["variant"][rows_idx])
            e_vr = (v - r_).abs().amax(-1)
        else:
            v1, e_vr = p1 * 0 - 1, pm * 0 - 1
        cols = torch.stack([p1.float(), r1.float(), t1.float(), rm, pm, tm, e_pr, e_pt, e_rt, gap, v1.float(), e_vr],
                           dim=1).cpu()
        for (row, request), c in zip(sampled, cols.tolist()):
            # a decode row becomes generated token g + 1; a last piece token 1
            k = request.generated_tokens + 1 if row >= len(plan.pieces) else 1
            report.rows.append(RowRecord(request.sequence_id, k, int(c[0]), int(c[1]), int(c[2]), c[3], c[4], c[5],
                                         c[6], c[7], c[8], c[9], int(c[10]), c[11]))
    report.sequences = {r.sequence_id: r.sequence for r in requests}
    return report
