"""Seeded synthetic inputs for the paged-attention benchmark workloads.

All values are drawn on the host with numpy's PCG64 (``default_rng(seed)``),
so every consumer — the HIP kernels, the reference-algorithm oracle and
the CPU baseline — sees bit-identical inputs.  Shapes follow the Llama-3.2-1B
attention geometry: 32 query heads, 8 KV heads, head_dim 64, block_size 16.

Workloads
  decode_small     4 sequences of {17, 64, 129, 500} tokens, pool of 256 blocks
  decode_ragged    16 sequences, lognormal lengths (median 2048, sigma 1,
                   clipped to [32, 29600]), pool = 2x the blocks needed
  mixed_prefill    4 prefill chunks of 128 tokens on contexts {0, 384, 1024,
                   4000} followed by 12 decode rows with contexts U[256, 8192]
  decode_long      16 sequences of 29600 tokens
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

Q_HEADS = 32
KV_HEADS = 8
HEAD_DIM = 64
BLOCK_SIZE = 16


@dataclass
class PagedWorkload:
    """A paged KV pool plus a ragged batch of new tokens to attend with."""

    num_layers: int
    num_blocks: int
    block_size: int
    q_heads: int
    kv_heads: int
    head_dim: int
    context_lens: list[int]          # tokens already cached per sequence
    query_lens: list[int]            # new tokens per sequence
    tables: list[list[int]]          # physical blocks per sequence (logical order)
    seed: int
    extra: dict = field(default_factory=dict)

    @property
    def seq_lens(self) -> list[int]:
        return [c + q for c, q in zip(self.context_lens, self.query_lens)]

    @property
    def num_tokens(self) -> int:
        return int(sum(self.query_lens))

    def slots(self) -> np.ndarray:
        out = []
        for table, ctx, q in zip(self.tables, self.context_lens, self.query_lens):
            pos = np.arange(ctx, ctx + q)
            out.append(np.asarray(table, dtype=np.int64)[pos // self.block_size] * self.block_size + pos % self.block_size)
        return np.concatenate(out) if out else np.zeros(0, dtype=np.int64)

    def table_array(self) -> np.ndarray:
        width = max(len(t) for t in self.tables)
        arr = np.zeros((len(self.tables), width), dtype=np.int32)
        for r, t in enumerate(self.tables):
            arr[r, : len(t)] = t
        return arr

    # -- value generation (host, fp32, then cast) -------------------------
    def pool(self, dtype: torch.dtype, device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
        """N(0,1) K and V pools (every slot filled, including unused ones)."""
        rng = np.random.default_rng(self.seed)
        shape = (self.num_layers, self.num_blocks, self.block_size, self.kv_heads, self.head_dim)
        k = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype)
        v = torch.from_numpy(rng.standard_normal(shape, dtype=np.float32)).to(dtype)
        return k.to(device), v.to(device)

    def new_tokens(self, dtype: torch.dtype, device="cpu") -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """N(0,1) queries (T, Hq, D) and new K/V rows (T, Hkv, D)."""
        rng = np.random.default_rng(self.seed + 1000)
        t = self.num_tokens
        q = rng.standard_normal((t, self.q_heads, self.head_dim), dtype=np.float32)
        k = rng.standard_normal((t, self.kv_heads, self.head_dim), dtype=np.float32)
        v = rng.standard_normal((t, self.kv_heads, self.head_dim), dtype=np.float32)
        return tuple(torch.from_numpy(x).to(dtype).to(device) for x in (q, k, v))  # type: ignore[return-value]


def _tables_from_permutation(rng: np.random.Generator, num_blocks: int, blocks_per_seq: list[int]) -> list[list[int]]:
    perm = rng.permutation(num_blocks)
    tables, cursor = [], 0
    for n in blocks_per_seq:
        tables.append([int(x) for x in perm[cursor : cursor + n]])
        cursor += n
    return tables


def ragged(
    context_lens: list[int],
    query_lens: list[int],
    *,
    seed: int,
    num_blocks: int | None = None,
    pool_factor: float = 2.0,
    num_layers: int = 1,
    q_heads: int = Q_HEADS,
    kv_heads: int = KV_HEADS,
    head_dim: int = HEAD_DIM,
    block_size: int = BLOCK_SIZE,
) -> PagedWorkload:
    """Generic workload: tables drawn from a seeded permutation of the pool."""
    rng = np.random.default_rng(seed)
    need = [-(-(c + q) // block_size) for c, q in zip(context_lens, query_lens)]
    if num_blocks is None:
        num_blocks = max(int(sum(need) * pool_factor), sum(need))
    tables = _tables_from_permutation(rng, num_blocks, need)
    return PagedWorkload(num_layers, num_blocks, block_size, q_heads, kv_heads, head_dim,
                         list(context_lens), list(query_lens), tables, seed)


def decode_small() -> PagedWorkload:
    """4 decode rows attending over {17, 64, 129, 500} cached tokens; 256-block pool, seed 0.

    The attended lengths include the current token, so contexts are length-1
    and each row appends one token.
    """
    lengths = [17, 64, 129, 500]
    return ragged([n - 1 for n in lengths], [1] * 4, seed=0, num_blocks=256)


def lognormal_lengths(seed: int = 1, count: int = 16) -> list[int]:
    rng = np.random.default_rng(seed)
    raw = rng.lognormal(mean=np.log(2048.0), sigma=1.0, size=count)
    return [int(x) for x in np.clip(np.round(raw), 32, 29600)]


def decode_ragged(num_layers: int = 1, seed: int = 1) -> PagedWorkload:
    """16 decode rows, lognormal contexts; pool = 2x the blocks needed."""
    ctx = lognormal_lengths(seed)
    return ragged(ctx, [1] * len(ctx), seed=seed, pool_factor=2.0, num_layers=num_layers)


def mixed_prefill(seed: int = 2) -> PagedWorkload:
    """4 x 128-token chunks on contexts {0, 384, 1024, 4000} + 12 decode rows."""
    rng = np.random.default_rng(seed + 77)
    decode_ctx = [int(x) for x in rng.integers(256, 8193, size=12)]
    return ragged([0, 384, 1024, 4000] + decode_ctx, [128] * 4 + [1] * 12, seed=seed, pool_factor=2.0)


def prefill_prompts(seed: int = 5) -> PagedWorkload:
    """4 fresh prompts of 2048 tokens each (no cached context), one chunk each."""
    return ragged([0] * 4, [2048] * 4, seed=seed, pool_factor=1.25)


def prefill_long_context(seed: int = 6) -> PagedWorkload:
    """4 chunks of 512 tokens on 8192-token cached contexts."""
    return ragged([8192] * 4, [512] * 4, seed=seed, pool_factor=1.25)


def decode_long(num_layers: int = 1, seed: int = 4, num_blocks: int | None = None) -> PagedWorkload:
    """16 decode rows at 29600 tokens of context (fully permuted tables)."""
    return ragged([29600] * 16, [1] * 16, seed=seed, num_blocks=num_blocks, pool_factor=2.0, num_layers=num_layers)


# ---------------------------------------------------------------------------
# End-to-end serving: the Llama-3.2-1B-shaped model and its request mix
# ---------------------------------------------------------------------------
SERVING_REQUESTS = 64
SERVING_NEW_TOKENS = 256
SERVING_MAX_BATCH = 16
SERVING_CHUNK = 128
SERVING_STEP_BUDGET = 512


def serving_model(device, seed: int = 3):
    """Llama-3.2-1B shape (``LlamaConfig`` defaults: hidden 2048, 16 layers,
    32 / 8 heads, MLP 8192, vocab 128256, tied embeddings), bf16, every
    Linear / Embedding weight N(0, 0.02), norm weights 1."""
    from torch import nn

    from nano_infer_engine.models.llama import Llama3_2, LlamaConfig

    torch.manual_seed(seed)
    with torch.device(device):
        model = Llama3_2(LlamaConfig())
    model = model.to(torch.bfloat16).eval()
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, 0.02)
    return model


def serving_prompts(device, vocab: int, count: int = SERVING_REQUESTS, seed: int = 3,
                    lengths: tuple[int, int] = (128, 2048)) -> list[torch.Tensor]:
    """``count`` prompts of token IDs uniform over the vocabulary, lengths
    uniform in ``lengths`` (inclusive), each (1, n) int64."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lengths[0], lengths[1] + 1, size=count)
    return [torch.from_numpy(rng.integers(0, vocab, size=(1, int(n)))).to(device) for n in lens]


def serving_cache_blocks(prompts, max_new_tokens: int, max_batch: int = SERVING_MAX_BATCH,
                         block_size: int = BLOCK_SIZE) -> int:
    """Pool blocks for a serving run: max_batch requests of the longest
    prompt at full length, plus 64 spare."""
    per_request = -(-(max(p.shape[1] for p in prompts) + max_new_tokens) // block_size)
    return max_batch * per_request + 64


# ---------------------------------------------------------------------------
# Algorithmic traffic / work (what roofline fractions are computed from)
# ---------------------------------------------------------------------------
def decode_bytes(seq_lens, q_heads=Q_HEADS, kv_heads=KV_HEADS, head_dim=HEAD_DIM, block_size=BLOCK_SIZE, elt=2) -> int:
    """sum_b [2*L_b*Hkv*D*s + 2*Hq*D*s + 4*ceil(L_b/BS) + 4]: K and V of every
    attended token, the query and output rows, the block-table entries and
    the length."""
    total = 0
    for n in seq_lens:
        total += 2 * n * kv_heads * head_dim * elt + 2 * q_heads * head_dim * elt + 4 * -(-n // block_size) + 4
    return total


def append_bytes(num_tokens, kv_heads=KV_HEADS, head_dim=HEAD_DIM, elt=2) -> int:
    """Each new token: read + write its K and V rows, and its 8-byte slot."""
    return num_tokens * (4 * kv_heads * head_dim * elt + 8)


def prefill_flops(context_lens, query_lens, q_heads=Q_HEADS, head_dim=HEAD_DIM) -> int:
    """4*Hq*D*sum_r [n_r*c_r + n_r(n_r+1)/2]: QK^T and PV over unmasked pairs."""
    pairs = sum(n * c + n * (n + 1) // 2 for c, n in zip(context_lens, query_lens))
    return 4 * q_heads * head_dim * pairs
