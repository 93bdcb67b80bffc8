"""Pins the oracle's whole-model restatement (``oracle.reference_model``) on the CPU.

``ReferenceLlama`` is the reference path the end-to-end greedy-identity
check compares the product against, so it is checked here against a float64
dense Llama forward written independently (numpy; attention through the
float64 closed form that ``test_oracle.py`` pins against brute force):
every packed token's logits in fp32 within 2e-4.  Chunked prefill over the
paged cache must equal the one-shot forward, and planted mistakes (a RoPE
sign, a dropped norm weight, a dropped residual) must fail the pin.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from nano_infer_engine.models.llama import Llama3_2, LlamaConfig
from nano_infer_engine.paged_cache import PagedKVCache
from oracle import closed_form, reference_model
from oracle.reference_ops import rope_module_inv_freq


def _model(seed=0):
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=96, hidden_size=64, mlp_inner_size=160, num_layers=2, q_head_num=4, kv_head_num=2,
                      rope_type="llama3", max_seq_len=256, tie_word_embeddings=True)
    model = Llama3_2(cfg).eval()
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "norm" in name or "rms" in name:
                p.copy_(1.0 + 0.2 * torch.randn_like(p))
            else:
                p.copy_(0.15 * torch.randn_like(p))
    return model


def _dense_float64(model, tokens: np.ndarray) -> np.ndarray:
    """Textbook Llama forward over one whole sequence in float64 (no cache)."""
    cfg = model.config
    f64 = lambda t: t.detach().double().numpy()  # noqa: E731
    hq, hkv, d = cfg.q_head_num, cfg.kv_head_num, cfg.head_dim
    inv = rope_module_inv_freq(model.rope, "cpu").double().numpy()
    pos = np.arange(len(tokens), dtype=np.float64)
    ang = pos[:, None] * inv[None, :]
    sin, cos = np.sin(ang)[:, None, :], np.cos(ang)[:, None, :]

    def norm(x, w, eps):
        return w * x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)

    def rope(x):
        a, b = x[..., : d // 2], x[..., d // 2 :]
        return np.concatenate([a * cos - b * sin, b * cos + a * sin], axis=-1)

    x = f64(model.embed.weight)[tokens]
    for block in model.decoders:
        at, ff = block.attn, block.ffn
        n = norm(x, f64(block.pre_norm.weight), block.pre_norm.eps)
        q = rope((n @ f64(at.q_proj.weight).T).reshape(-1, hq, d))
        k = rope((n @ f64(at.k_proj.weight).T).reshape(-1, hkv, d))
        v = (n @ f64(at.v_proj.weight).T).reshape(-1, hkv, d)
        ctx = closed_form.attention(q, k, v, list(range(len(tokens))), d**-0.5).reshape(len(tokens), hq * d)
        h = ctx @ f64(at.o_proj.weight).T + x
        m = norm(h, f64(block.post_norm.weight), block.post_norm.eps)
        g = m @ f64(ff.gate_proj.weight).T
        x = ((g / (1 + np.exp(-g))) * (m @ f64(ff.up_proj.weight).T)) @ f64(ff.down_proj.weight).T + h
    x = norm(x, f64(model.final_rms.weight), model.final_rms.eps)
    return x @ f64(model.lm_head.weight).T


def _cache(model, dtype=torch.float32):
    cfg = model.config
    return PagedKVCache(64, 4, cfg.num_layers, cfg.kv_head_num, cfg.head_dim, dtype, "cpu")


def _prompts():
    rng = np.random.default_rng(7)
    return [rng.integers(0, 96, size=n) for n in (13, 5, 22)]


def _ragged_logits(model, prompts, chunk):
    """ReferenceLlama over the prompts in ragged steps of at most ``chunk`` tokens each."""
    ref = reference_model.ReferenceLlama(model, torch.float32)
    cache = _cache(model)
    ids = tuple(f"s{i}" for i in range(len(prompts)))
    done = [0] * len(prompts)
    out = [[] for _ in prompts]
    while any(done[i] < len(p) for i, p in enumerate(prompts)):
        live = [i for i, p in enumerate(prompts) if done[i] < len(p)]
        pieces = [prompts[i][done[i] : done[i] + chunk] for i in live]
        bounds = np.cumsum([0] + [len(p) for p in pieces]).tolist()
        logits = ref.forward_ragged(torch.from_numpy(np.concatenate(pieces)), kv_cache=cache,
                                    sequence_ids=tuple(ids[i] for i in live), query_start_loc=bounds)
        for j, i in enumerate(live):
            out[i].append(logits[bounds[j] : bounds[j + 1]].double().numpy())
            done[i] += len(pieces[j])
    return [np.concatenate(rows) for rows in out]


@pytest.mark.parametrize("chunk", [64, 4])
def test_reference_model_matches_dense_float64(chunk):
    model = _model()
    prompts = _prompts()
    got = _ragged_logits(model, prompts, chunk)
    for p, g in zip(prompts, got):
        want = _dense_float64(model, p)
        err = np.abs(g - want).max()
        assert err < 2e-4, err


@pytest.mark.parametrize("kind", ["rope_sign", "norm_weight", "residual"])
def test_reference_model_pin_catches_planted_mistakes(kind, monkeypatch):
    model = _model()
    if kind == "rope_sign":
        def bad_rope(x, sin, cos):  # rotation by -angle
            first, second = x.chunk(2, dim=-1)
            sin, cos = sin[:, None, :], cos[:, None, :]
            return torch.cat((first * cos + second * sin, second * cos - first * sin), dim=-1)
        monkeypatch.setattr(reference_model, "rope_rotate", bad_rope)
    elif kind == "norm_weight":
        monkeypatch.setattr(reference_model, "rms_norm_reference",
                            lambda x, w, eps: (x.float() / torch.sqrt(x.float().pow(2).mean(-1, keepdim=True) + eps))
                            .to(x.dtype))
    else:
        original = reference_model.ReferenceLlama._attention

        def no_residual(self, x, *args):
            return original(self, x, *args) - x  # the caller adds x back: net effect drops the residual

        monkeypatch.setattr(reference_model.ReferenceLlama, "_attention", no_residual)
    prompts = _prompts()
    got = _ragged_logits(model, prompts, 64)
    err = max(np.abs(g - _dense_float64(model, p)).max() for p, g in zip(prompts, got))
    assert err > 1e-2, (kind, err)


def test_reference_model_bf16_close_to_float64():
    """The bf16 restatement stays within bf16 rounding of the truth on this small model."""
    model = _model()
    ref = reference_model.ReferenceLlama(model, torch.bfloat16)
    cache = _cache(model, torch.bfloat16)
    p = _prompts()[2]
    got = ref.forward_ragged(torch.from_numpy(p), kv_cache=cache, sequence_ids=("s",), query_start_loc=[0, len(p)])
    want = _dense_float64(model, p)
    err = np.abs(got.double().numpy() - want).max()
    assert err < 0.1 * np.abs(want).max(), err
