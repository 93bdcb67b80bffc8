from nano_infer_engine.models.llama import Llama3_2, LlamaConfig, RopeScalingConfig

__all__ = ["Llama3_2", "LlamaConfig", "RopeScalingConfig"]
