"""CPU restatement of ``resident_epoch_execute``'s host-side packing.

Oracle (test infrastructure only).  Restates
native/resident_epoch_bridge.cpp ("BRIDGE") for B rows:

* ``bridge_compute_slot`` -- BRIDGE:350-357 (row r owns blocks r*BPR..).
* ``execute``             -- BRIDGE:424-649 without the import paths: argument
  validation (status 10/11/12), the identity block table (524-526), the 260-byte
  feed for B=4 (499-569), the control vector with the configured EOS 151645
  for empty rows (555-567), and the unpacking of the fetched history
  ``[step][row]`` into ``tokens[row*8+step]`` (617-642).

Parity pinning: known-answer cases computed by hand from the closed forms
(tests/test_oracle_bridge.py) and the byte ledger of
src/vllm_ascend_resident_epoch/abi.py:18-76 (260/368 bytes).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .controller import EpochController, EpochFeed, MAX_EPOCH_STEPS

CONFIGURED_EOS = 151645  # BRIDGE:31
COMMIT_PREPARED, COMMIT_EXECUTING, COMMIT_COMMITTED = 0, 1, 2  # PROTO.h:23-25


def bridge_compute_slot(row: int, position: int, batch: int, capacity: int, blocks_per_row: int, block_size: int) -> int:
    """BRIDGE:350-357."""
    if row < 0 or row >= batch or position < 0 or position >= capacity:
        return -1
    return row * blocks_per_row * block_size + position


def feed_bytes(batch: int, blocks_per_row: int) -> int:
    """Declared feed size: token, position, length, slot, active, table,
    tiling, control (BRIDGE:53-62; abi.py:18-27)."""
    return 8 * batch + 8 * batch + 4 * batch + 4 * batch + 4 * batch + 4 * batch * blocks_per_row + 72 + 4 * (3 + 2 * batch)


def fetch_bytes(batch: int) -> int:
    """Declared fetch size: history int64[8,B] and control int32[6+4B+2+B]."""
    return 8 * MAX_EPOCH_STEPS * batch + 4 * (6 + 4 * batch + 2 + batch)


@dataclass
class BridgeResult:
    status: int
    commit_state: int
    token_ids: np.ndarray  # int64 [B*8]
    executed: np.ndarray  # int32 [B]
    row_generations: np.ndarray  # int32 [B]
    model_calls: int = 0
    device_status: int = -1
    feed_calls: int = 0
    fetch_calls: int = 0
    declared_input_bytes: int = 0
    declared_output_bytes: int = 0


def execute(
    controller: EpochController,
    request_count: int,
    max_steps: int,
    tokens,
    positions,
    lengths,
    eos,
    generations,
    tiling: bytes,
    configured_eos: int = CONFIGURED_EOS,
) -> BridgeResult:
    """BRIDGE:424-649 (non-import path).

    ``configured_eos`` is the EOS id fed for empty rows (BRIDGE:31 hard-codes
    the 7B id 151645, which is out of range for the tiny 4096-entry vocab).
    """
    g = controller.geometry
    B = g.batch
    out_tokens = np.full(B * MAX_EPOCH_STEPS, -1, dtype=np.int64)
    out_exec = np.zeros(B, dtype=np.int32)
    out_gen = np.zeros(B, dtype=np.int32)
    result = BridgeResult(10, COMMIT_PREPARED, out_tokens, out_exec, out_gen)
    if request_count < 1 or request_count > B or max_steps < 1 or max_steps > MAX_EPOCH_STEPS:
        return result  # BRIDGE:443-459
    result.declared_input_bytes = feed_bytes(B, g.blocks_per_row)
    result.declared_output_bytes = fetch_bytes(B)
    table = np.zeros(B * g.blocks_per_row, dtype=np.int32)
    tok = np.zeros(B, dtype=np.int64)
    pos = np.zeros(B, dtype=np.int64)
    length = np.zeros(B, dtype=np.int32)
    slot = np.zeros(B, dtype=np.int32)
    active = np.zeros(B, dtype=np.int32)
    for r in range(B):  # BRIDGE:524-532
        for j in range(g.blocks_per_row):
            table[r * g.blocks_per_row + j] = r * g.blocks_per_row + j
        slot[r] = bridge_compute_slot(r, 0, B, g.capacity, g.blocks_per_row, g.block_size)
    active_count = 0
    for r in range(B):  # BRIDGE:533-551
        if int(generations[r]) == 0:
            continue
        active_count += 1
        if (
            int(generations[r]) < 0
            or int(tokens[r]) < 0
            or int(tokens[r]) >= g.vocab
            or int(positions[r]) < 0
            or int(positions[r]) + max_steps > g.capacity
            or int(lengths[r]) != int(positions[r]) + 1
            or int(eos[r]) < 0
            or int(eos[r]) >= g.vocab
        ):
            result.status = 11
            return result
        tok[r] = int(tokens[r])
        pos[r] = int(positions[r])
        length[r] = int(lengths[r])
        slot[r] = bridge_compute_slot(r, int(positions[r]), B, g.capacity, g.blocks_per_row, g.block_size)
        active[r] = 1
    if active_count != request_count:
        result.status = 12
        return result
    control = np.zeros(3 + 2 * B, dtype=np.int32)  # BRIDGE:555-567
    control[0] = max_steps
    for r in range(B):
        control[1 + r] = int(eos[r]) if int(generations[r]) != 0 else configured_eos
        control[3 + B + r] = int(generations[r])
    result.commit_state = COMMIT_EXECUTING
    fetch = controller.proc(EpochFeed(tok, pos, length, slot, active, table, tiling, control))
    result.feed_calls = 1
    result.fetch_calls = 1
    result.device_status = int(fetch.control[3])
    result.model_calls = int(fetch.control[4])
    for r in range(B):  # BRIDGE:632-642
        executed = int(fetch.control[g.executed_off + r])
        if executed < 0 or executed > max_steps:
            result.status = 33
            return result
        out_exec[r] = executed
        out_gen[r] = int(fetch.control[g.generation_off + r])
        for s in range(executed):
            out_tokens[r * MAX_EPOCH_STEPS + s] = fetch.history[s, r]
    result.commit_state = COMMIT_COMMITTED
    result.status = 0
    return result
