"""Scheduler-side configuration of resident epochs.

Mirrors src/vllm_ascend_resident_epoch/config.py:16-42: epoch length K and
logical capacity from the environment, the paged geometry of the B=4 graph.
"""
from __future__ import annotations

import os
from dataclasses import dataclass

EPOCH_STEP_CHOICES = (1, 2, 4, 8)


def _env_int(name: str, default: int) -> int:
    raw = os.getenv(name)
    if raw is None:
        return default
    try:
        return int(raw)
    except ValueError as exc:
        raise ValueError(f"{name} must be an integer, got {raw!r}") from exc


@dataclass(frozen=True)
class ResidentEpochConfig:
    max_steps: int = 8
    logical_capacity: int = 8
    physical_blocks: int = 8
    blocks_per_request: int = 2
    block_size: int = 128
    max_batch_size: int = 4

    @classmethod
    def from_env(cls) -> "ResidentEpochConfig":
        config = cls(
            max_steps=_env_int("VLLM_ASCEND_RESIDENT_EPOCH_STEPS", 8),
            logical_capacity=_env_int("VLLM_ASCEND_RESIDENT_EPOCH_CAPACITY", 8),
        )
        config.validate()
        return config

    def validate(self) -> None:
        if self.max_steps not in EPOCH_STEP_CHOICES:
            raise ValueError("resident epoch steps must be one of 1, 2, 4, 8")
        if self.logical_capacity < self.max_steps:
            raise ValueError("logical capacity must be at least max_steps")
        if self.max_batch_size != 4:
            raise ValueError("the current native graph has a fixed maximum B=4")
