from nano_infer_engine.layers.attention import GroupedQueryAttention
from nano_infer_engine.layers.decoder import Llama3Decoder
from nano_infer_engine.layers.mlp import SwiGLUMLP
from nano_infer_engine.layers.paged_attention import (
    batched_paged_attention_reference,
    paged_attention_reference,
)
from nano_infer_engine.layers.rms_norm import RmsNorm
from nano_infer_engine.layers.rope import Rope, RopeScale

__all__ = [
    "GroupedQueryAttention",
    "Llama3Decoder",
    "RmsNorm",
    "Rope",
    "RopeScale",
    "SwiGLUMLP",
    "batched_paged_attention_reference",
    "paged_attention_reference",
]
