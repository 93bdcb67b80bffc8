"""Request state of the continuous-batching scheduler (``generation/request.py:7-34`` of the reference)."""

from dataclasses import dataclass, field
from enum import Enum

import torch


class RequestStatus(str, Enum):
    PENDING = "pending"
    PREFILLING = "prefilling"
    ACTIVE = "active"
    COMPLETED = "completed"
    FAILED = "failed"
    CANCELLED = "cancelled"


@dataclass
class PagedRequest:
    sequence_id: str
    prompt: torch.Tensor
    generated_tokens: int = 0
    finished: bool = False
    required_blocks: int = 0
    last_logits: torch.Tensor | None = None
    prefill_offset: int = 0
    status: RequestStatus = RequestStatus.PENDING
    error: Exception | None = None
    # the prompt and the tokens generated so far: a joined (1, n) prefix plus
    # tokens not yet joined (see `sequence`): (1, 1) tensors, or (tokens,
    # row) pairs naming row `row` of a step's (n, 1) tokens
    _joined: torch.Tensor | None = field(init=False, default=None, repr=False, compare=False)
    _pending: list = field(init=False, default_factory=list, repr=False, compare=False)

    def __post_init__(self) -> None:
        self._joined = self.prompt

    @property
    def sequence(self) -> torch.Tensor:
        """The prompt followed by the generated tokens, (1, length).

        Tokens appended by the scheduler are joined when this is read, in one
        concatenation, instead of one device copy per token and step.
        """
        if self._pending:
            parts = [p if isinstance(p, torch.Tensor) else p[0][p[1] : p[1] + 1] for p in self._pending]
            self._joined = torch.cat((self._joined, *parts), dim=1)
            self._pending = []
        return self._joined

    @sequence.setter
    def sequence(self, value: torch.Tensor) -> None:
        self._joined = value
        self._pending = []

    def append_token(self, token: torch.Tensor) -> None:
        """Appends a generated token, a (1, 1) tensor (kept as given until `sequence` is read)."""
        self._pending.append(token)

    def _append_row(self, tokens: torch.Tensor, row: int) -> None:
        """Appends row ``row`` of a step's (n, 1) tokens, sliced only when
        `sequence` is read (a decode step's requests each take one row)."""
        self._pending.append((tokens, row))
