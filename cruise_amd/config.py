"""Geometry and epoch length of the resident graph, as the scheduler sees it.

The field names, their defaults and the two environment variables are the
reference's interface (src/vllm_ascend_resident_epoch/config.py:16-33): K
from VLLM_ASCEND_RESIDENT_EPOCH_STEPS, the logical capacity from
VLLM_ASCEND_RESIDENT_EPOCH_CAPACITY, and the B=4 paged geometry (2 blocks of
128 tokens per row).  The same three limits hold (config.py:35-42): K is a
power of two up to 8, the capacity covers one full epoch, and the graph has
four rows.  This module also owns the two derived rules every caller of the
geometry needs: which device blocks a row owns, and the K of an epoch under a
step budget.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, fields
from typing import Mapping

EPOCH_STEP_CHOICES = (1, 2, 4, 8)
GRAPH_ROWS = 4

# configuration field -> environment variable that overrides it
ENVIRONMENT = {
    "max_steps": "VLLM_ASCEND_RESIDENT_EPOCH_STEPS",
    "logical_capacity": "VLLM_ASCEND_RESIDENT_EPOCH_CAPACITY",
}


def epoch_steps_within(budget: int) -> int:
    """The largest allowed epoch length that fits ``budget`` steps
    (scheduler.py:244-247); ``budget`` must be at least 1."""
    if budget < 1:
        raise ValueError("an epoch needs a budget of at least one step")
    return max(k for k in EPOCH_STEP_CHOICES if k <= budget)


@dataclass(frozen=True)
class ResidentEpochConfig:
    max_steps: int = 8
    logical_capacity: int = 8
    physical_blocks: int = 8
    blocks_per_request: int = 2
    block_size: int = 128
    max_batch_size: int = 4

    @classmethod
    def from_env(cls, environ: Mapping[str, str] | None = None) -> "ResidentEpochConfig":
        """The defaults overridden by the environment (or ``environ``);
        raises ValueError on a non-integer value or a violated limit."""
        env = os.environ if environ is None else environ
        overrides = {}
        for name, variable in ENVIRONMENT.items():
            text = env.get(variable)
            if text is None:
                continue
            try:
                overrides[name] = int(text)
            except ValueError:
                raise ValueError(f"{variable}={text!r} is not an integer") from None
        config = cls(**overrides)
        config.validate()
        return config

    def problems(self) -> list[str]:
        """Every violated limit, in words; empty when the configuration can
        run on the graph."""
        found = []
        if self.max_steps not in EPOCH_STEP_CHOICES:
            found.append(f"max_steps={self.max_steps} is not one of {EPOCH_STEP_CHOICES}")
        if self.logical_capacity < self.max_steps:
            found.append(f"logical_capacity={self.logical_capacity} cannot hold an epoch of {self.max_steps} steps")
        if self.max_batch_size != GRAPH_ROWS:
            found.append(f"max_batch_size={self.max_batch_size}: the graph is built for exactly {GRAPH_ROWS} rows")
        return found

    def validate(self) -> None:
        found = self.problems()
        if found:
            raise ValueError("resident epoch configuration: " + "; ".join(found))

    def row_blocks(self, row: int) -> tuple[int, ...]:
        """Device blocks of a graph row: row r owns the consecutive run
        starting at r * blocks_per_request."""
        first = row * self.blocks_per_request
        return tuple(range(first, first + self.blocks_per_request))

    def epoch_steps(self, budget: int) -> int:
        """K of an epoch that may run at most ``budget`` steps under this
        configuration's max_steps."""
        return epoch_steps_within(min(budget, self.max_steps))

    def as_dict(self) -> dict[str, int]:
        return {f.name: getattr(self, f.name) for f in fields(self)}
