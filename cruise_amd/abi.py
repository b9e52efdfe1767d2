"""Byte ledger of the epoch ABI.

The reference moved from a decoder-shaped epoch ABI (the KV caches and the
full logits history crossed the host boundary every epoch) to the resident
one (8 small inputs, 2 small outputs; src/vllm_ascend_resident_epoch/
abi.py:18-76).  This module states both as tensor specs, derived from the
geometry so the same ledger covers the scaled configurations, and checks the
reference's totals for the Qwen2.5-7B B=4 geometry at import time.
"""
from __future__ import annotations

from dataclasses import dataclass
from math import prod


@dataclass(frozen=True)
class TensorSpec:
    name: str
    shape: tuple[int, ...]
    element_bytes: int

    @property
    def nbytes(self) -> int:
        return prod(self.shape) * self.element_bytes


@dataclass(frozen=True)
class EpochGeometry:
    """Shapes that size the epoch's tensors (Qwen2.5-7B B=4 by default)."""

    batch: int = 4
    blocks_per_row: int = 2
    layers: int = 28
    physical_blocks: int = 8
    block_size: int = 128
    kv_heads: int = 4
    head_dim: int = 128
    vocab: int = 152064
    max_steps: int = 8
    element_bytes: int = 2


def common_inputs(g: EpochGeometry = EpochGeometry()) -> tuple[TensorSpec, ...]:
    """The eight inputs of the resident epoch, in feed order."""
    return (
        TensorSpec("token", (g.batch, 1), 8),
        TensorSpec("position", (g.batch,), 8),
        TensorSpec("sequence_length", (g.batch, 1), 4),
        TensorSpec("slot_mapping", (g.batch,), 4),
        TensorSpec("active_mask", (g.batch,), 4),
        TensorSpec("block_table", (g.batch, g.blocks_per_row), 4),
        TensorSpec("tiling", (72,), 1),
        TensorSpec("control", (3 + 2 * g.batch,), 4),
    )


def cache_spec(name: str, g: EpochGeometry = EpochGeometry()) -> TensorSpec:
    return TensorSpec(name, (g.layers, g.physical_blocks, g.block_size, g.kv_heads, g.head_dim), g.element_bytes)


def resident_outputs(g: EpochGeometry = EpochGeometry()) -> tuple[TensorSpec, ...]:
    return (
        TensorSpec("token_history", (g.max_steps, g.batch), 8),
        TensorSpec("control_output", (6 + 4 * g.batch + 2 + g.batch,), 4),
    )


def decoder_shaped_inputs(g: EpochGeometry = EpochGeometry()) -> tuple[TensorSpec, ...]:
    """The decoder-shaped epoch: the common inputs with both caches inserted
    in the decoder's argument order."""
    c = common_inputs(g)
    return c[:3] + (cache_spec("key_cache", g),) + c[3:6] + (cache_spec("value_cache", g),) + c[6:]


def decoder_shaped_outputs(g: EpochGeometry = EpochGeometry()) -> tuple[TensorSpec, ...]:
    hist, control = resident_outputs(g)
    return (
        TensorSpec("logits_history", (g.max_steps, g.batch, 1, g.vocab), 4),
        hist,
        cache_spec("key_cache", g),
        cache_spec("value_cache", g),
        TensorSpec("final_token", (g.batch, 1), 8),
        TensorSpec("final_position", (g.batch,), 8),
        TensorSpec("final_length", (g.batch, 1), 4),
        TensorSpec("final_slot", (g.batch,), 4),
        TensorSpec("final_active", (g.batch,), 4),
        control,
    )


def total_bytes(specs: tuple[TensorSpec, ...]) -> int:
    return sum(s.nbytes for s in specs)


COMMON_INPUTS = common_inputs()
KEY_CACHE = cache_spec("key_cache")
VALUE_CACHE = cache_spec("value_cache")
TOKEN_HISTORY, CONTROL_OUTPUT = resident_outputs()
OLD_INPUTS = decoder_shaped_inputs()
OLD_OUTPUTS = decoder_shaped_outputs()
NEW_INPUTS = COMMON_INPUTS
NEW_OUTPUTS = resident_outputs()

ABI_BYTES = {
    "old": {"input": total_bytes(OLD_INPUTS), "output": total_bytes(OLD_OUTPUTS)},
    "new": {"input": total_bytes(NEW_INPUTS), "output": total_bytes(NEW_OUTPUTS)},
}
OLD_TOTAL_BYTES = ABI_BYTES["old"]["input"] + ABI_BYTES["old"]["output"]
NEW_TOTAL_BYTES = ABI_BYTES["new"]["input"] + ABI_BYTES["new"]["output"]
TOTAL_REDUCTION_BYTES = OLD_TOTAL_BYTES - NEW_TOTAL_BYTES
KV_ROUND_TRIP_BYTES = 2 * (KEY_CACHE.nbytes + VALUE_CACHE.nbytes)

# The reference's ledger for Qwen2.5-7B B=4 (abi.py:73-76).
assert ABI_BYTES["old"] == {"input": 58_720_516, "output": 78_184_928}
assert ABI_BYTES["new"] == {"input": 260, "output": 368}
assert TOTAL_REDUCTION_BYTES == 136_904_816
assert KV_ROUND_TRIP_BYTES == 117_440_512
