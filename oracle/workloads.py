"""The five workload configurations (shapes, seeds, prompts, budgets).

Oracle (test infrastructure only).  C1 tiny fp32 model; C2 one Qwen2.5-7B
layer in bf16 over a 64-block pool; C3 the full Qwen2.5-7B shape; C4 the
multi-epoch cohort on the C2 model (run_multi_epoch_cohort.py:128-278 and
verify_multi_epoch_cohort_result.py:29-63 pin its row/generation structure);
C5 the B=64 scaled batch.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .decoder import ModelDims, PagedGeometry

C1_DIMS = ModelDims(
    num_layers=2, hidden=256, num_heads=4, num_kv_heads=2, head_dim=64, intermediate=688, vocab=4096, dtype="fp32"
)
C2_DIMS = ModelDims(
    num_layers=1, hidden=3584, num_heads=28, num_kv_heads=4, head_dim=128, intermediate=18944, vocab=152064, dtype="bf16"
)
C3_DIMS = ModelDims(
    num_layers=28, hidden=3584, num_heads=28, num_kv_heads=4, head_dim=128, intermediate=18944, vocab=152064, dtype="bf16"
)


@dataclass(frozen=True)
class Workload:
    name: str
    dims: ModelDims
    geometry: PagedGeometry
    eos: int
    seed: int


C1 = Workload("tiny-fp32", C1_DIMS, PagedGeometry(batch=4, physical_blocks=8, block_size=16, blocks_per_row=2, window=32), eos=4095, seed=20261)
C2 = Workload("qwen7b-1layer", C2_DIMS, PagedGeometry(batch=4, physical_blocks=64, block_size=128, blocks_per_row=2, window=256), eos=151645, seed=20262)
C3 = Workload("qwen7b", C3_DIMS, PagedGeometry(batch=4, physical_blocks=8, block_size=128, blocks_per_row=2, window=256), eos=151645, seed=20263)
C5 = Workload("qwen7b-1layer-b64", C2_DIMS, PagedGeometry(batch=64, physical_blocks=1024, block_size=128, blocks_per_row=8, window=1024), eos=151645, seed=20265)


def prompts(rng: np.random.Generator, batch: int, vocab: int, low: int = 2, high: int = 5) -> list[list[int]]:
    """Prompt ids uniform in [0, vocab) with lengths uniform in [low, high]."""
    return [list(map(int, rng.integers(0, vocab, size=int(rng.integers(low, high + 1))))) for _ in range(batch)]


def budgets(rng: np.random.Generator, batch: int, low: int = 2, high: int = 5) -> list[int]:
    return [int(v) for v in rng.integers(low, high + 1, size=batch)]


def random_tables(rng: np.random.Generator, batch: int, blocks_per_row: int, pool: int) -> np.ndarray:
    """Distinct physical blocks for every (row, logical block) from the pool."""
    picks = rng.choice(pool, size=batch * blocks_per_row, replace=False)
    return picks.astype(np.int32).reshape(batch, blocks_per_row)


def identity_table(batch: int, blocks_per_row: int) -> np.ndarray:
    """Row r owns blocks r*BPR .. r*BPR+BPR-1 (native/resident_epoch_bridge.cpp:524-526)."""
    return np.arange(batch * blocks_per_row, dtype=np.int32).reshape(batch, blocks_per_row)


def slot_of(table: np.ndarray, row: int, position: int, block_size: int) -> int:
    return int(table[row, position // block_size]) * block_size + position % block_size
