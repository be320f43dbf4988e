"""Per-request sampling parameters.

Same fields, types and defaults as the reference's ``SamplingParams``
(nanoserve/config.py:68-79), so request objects built by the reference's API
layer (nanoserve/api/server.py:51-67) can be handed to this sampler unchanged.
The sampler reads ``temperature``, ``top_p``, ``top_k`` and
``repetition_penalty``, and ``seed`` when no uniforms are passed: a seeded row
draws a Philox4x32-10 uniform keyed by the seed and counted by the row's
history length (the reference declares ``seed`` but never reads it).
``max_tokens``, ``stop_token_ids``, ``stop`` and ``ignore_eos`` belong to the
scheduler (nanoserve/scheduler/scheduler.py:295-306).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional


@dataclass
class SamplingParams:
    """Per-request sampling configuration (nanoserve/config.py:68-79)."""

    max_tokens: int = 128
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = -1
    repetition_penalty: float = 1.0
    stop_token_ids: list = field(default_factory=list)
    stop: list = field(default_factory=list)
    ignore_eos: bool = False
    seed: Optional[int] = None
