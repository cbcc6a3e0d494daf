"""Per-request sampling parameters: the worker protocol's `Sampling` object (volundr-mlx/session.py:439-478).

Same fields, defaults and predicates as the reference, so requests built for it work unchanged here.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional


@dataclass
class Sampling:
    """The worker protocol's sampling object (agens-server SamplingParams); session.py:439-456."""
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: Optional[int] = None
    min_p: float = 0.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    min_new_tokens: int = 0
    max_new_tokens: int = 256
    seed: Optional[int] = None
    logit_bias: list = field(default_factory=list)  # [(id, bias)]
    suppress_tokens: list = field(default_factory=list)
    stop_token_ids: list = field(default_factory=list)
    ignore_eos: bool = False
    reasoning_budget: Optional[int] = None
    reasoning_budget_soft_bias: float = 0.0

    @classmethod
    def from_dict(cls, d: dict):
        """session.py:458-463: unknown keys and None values are dropped; logit_bias becomes [(int, float)]."""
        names = cls.__dataclass_fields__.keys()
        s = cls(**{k: v for k, v in (d or {}).items() if k in names and v is not None})
        s.logit_bias = [(int(t), float(b)) for t, b in s.logit_bias]
        return s

    @property
    def greedy(self) -> bool:
        """session.py:466-467."""
        return self.top_k == 1 or self.temperature < 1e-6

    def needs_logits(self, vocab_valid: int, produced: int = 0) -> bool:
        """session.py:469-474: anything beyond an argmax over the valid vocabulary."""
        return (not self.greedy or bool(self.logit_bias) or self.repetition_penalty != 1.0
                or self.frequency_penalty != 0.0 or self.presence_penalty != 0.0
                or (produced < self.min_new_tokens and bool(self.stop_token_ids))
                or any(t < vocab_valid for t in self.suppress_tokens))

    def speculative(self, vocab_valid: int) -> bool:
        """session.py:476-478: greedy requests decode speculatively."""
        return self.greedy and not self.needs_logits(vocab_valid) and self.reasoning_budget is None
