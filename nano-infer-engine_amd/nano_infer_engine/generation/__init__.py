from nano_infer_engine.generation.config import GenerationConfig, GenerationOutput, RaggedGenerationOutput
from nano_infer_engine.generation.events import RequestResult, SchedulerStepOutput, TokenEvent
from nano_infer_engine.generation.paged_greedy import paged_greedy_generate
from nano_infer_engine.generation.paged_prefill import paged_prefill, paged_prefill_chunks
from nano_infer_engine.generation.request import PagedRequest, RequestStatus
from nano_infer_engine.generation.scheduler import ContinuousBatchingScheduler

__all__ = [
    "ContinuousBatchingScheduler",
    "GenerationConfig",
    "GenerationOutput",
    "PagedRequest",
    "RaggedGenerationOutput",
    "RequestResult",
    "RequestStatus",
    "SchedulerStepOutput",
    "TokenEvent",
    "paged_greedy_generate",
    "paged_prefill",
    "paged_prefill_chunks",
]
