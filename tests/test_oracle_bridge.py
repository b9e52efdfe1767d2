"""The bridge oracle against hand-derived known answers (CPU only).

native/resident_epoch_bridge.cpp ("BRIDGE"): argument checks 443-459 (status
10), per-row checks 533-551 (11), active-count check 552-553 (12), the
identity block table and slots 524-532 (row r owns blocks r*BPR..), the
control vector with the configured EOS for empty rows 555-567, and the
unpacking of history [step][row] into tokens[row*8 + step] 617-642.  Byte
sizes against the reference's ABI ledger
(src/vllm_ascend_resident_epoch/abi.py:18-76: 260 bytes in, 368 out).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bridge import (
    COMMIT_COMMITTED,
    COMMIT_EXECUTING,
    COMMIT_PREPARED,
    CONFIGURED_EOS,
    bridge_compute_slot,
    execute,
    feed_bytes,
    fetch_bytes,
)
from oracle.controller import ControllerGeometry, EpochController

B, V = 4, 64
GEO = ControllerGeometry(batch=B, capacity=8, physical_blocks=8, blocks_per_row=2, block_size=4, vocab=V, num_layers=1)
TILING = bytes(72)


def successor(token: int) -> int:
    return (3 * token + 1) % V


class Stub:
    def __call__(self, token, position, length, table, slot, key, value, tiling, active, *, inplace=False):
        logits = torch.zeros(B, 1, V)
        for r in range(B):
            logits[r, 0, successor(int(token[r, 0]))] = 1.0
        return logits, key, value, torch.where(active.to(torch.bool), position + 1, position)


class Recorder:
    """Controller stand-in: records each feed, then runs the oracle controller."""

    def __init__(self):
        self.geometry = GEO
        self.inner = EpochController(GEO, Stub(), (1, GEO.physical_blocks, GEO.block_size, 1, 2), torch.float32)
        self.feeds = []

    def proc(self, feed):
        self.feeds.append(feed)
        return self.inner.proc(feed)


def run(request_count=2, max_steps=3, tokens=(5, 6, 0, 0), positions=(0, 0, 0, 0), lengths=(1, 1, 0, 0),
        eos=(V - 1, V - 1, 0, 0), gens=(1, 2, 0, 0), configured_eos=V - 1):
    rec = Recorder()
    res = execute(rec, request_count, max_steps, tokens, positions, lengths, eos, gens, TILING, configured_eos=configured_eos)
    return rec, res


def test_declared_bytes_match_reference_abi_ledger():
    assert feed_bytes(4, 2) == 260
    assert fetch_bytes(4) == 368
    assert CONFIGURED_EOS == 151645


def test_bridge_slot_closed_form():
    # BRIDGE:350-357: row r owns slots r*BPR*bs .. ; out-of-range -> -1
    assert bridge_compute_slot(2, 5, 4, 256, 2, 128) == 2 * 2 * 128 + 5
    assert bridge_compute_slot(0, 256, 4, 256, 2, 128) == -1
    assert bridge_compute_slot(4, 0, 4, 256, 2, 128) == -1
    assert bridge_compute_slot(-1, 0, 4, 256, 2, 128) == -1


@pytest.mark.parametrize("request_count,max_steps", [(0, 3), (5, 3), (2, 0), (2, 9)])
def test_status_10_bad_arguments(request_count, max_steps):
    rec, res = run(request_count=request_count, max_steps=max_steps)
    assert res.status == 10 and res.commit_state == COMMIT_PREPARED
    assert rec.feeds == [] and (res.token_ids == -1).all()


@pytest.mark.parametrize(
    "field,value",
    [
        ("tokens", (5, V, 0, 0)),
        ("tokens", (-1, 6, 0, 0)),
        ("positions", (6, 0, 0, 0)),  # 6 + 3 > capacity 8
        ("lengths", (2, 1, 0, 0)),
        ("eos", (V, V - 1, 0, 0)),
        ("gens", (-3, 2, 0, 0)),
    ],
)
def test_status_11_bad_row(field, value):
    kwargs = {field: value}
    if field == "positions":
        kwargs["lengths"] = (7, 1, 0, 0)
    rec, res = run(**kwargs)
    assert res.status == 11 and res.commit_state == COMMIT_PREPARED and rec.feeds == []


def test_status_12_active_count_mismatch():
    rec, res = run(request_count=3)
    assert res.status == 12 and rec.feeds == []


def test_device_fallback_passes_through_with_status_0():
    # a new generation must start at position 0 (CTRL:461-468): device status
    # 212; the bridge still commits and returns 0 (BRIDGE:621-648)
    rec, res = run(tokens=(5, 6, 0, 0), positions=(2, 0, 0, 0), lengths=(3, 1, 0, 0))
    assert res.status == 0 and res.device_status == 212 and res.commit_state == COMMIT_COMMITTED
    assert res.model_calls == 0 and list(res.executed) == [0] * B and (res.token_ids == -1).all()


def test_feed_packing_and_unpacking():
    rec, res = run(tokens=(5, 6, 0, 0), positions=(0, 0, 0, 0), lengths=(1, 1, 0, 0), gens=(1, 2, 0, 0), configured_eos=33)
    assert res.status == 0 and res.commit_state == COMMIT_COMMITTED
    feed = rec.feeds[0]
    assert list(feed.block_table) == list(range(B * GEO.blocks_per_row))  # identity table
    # every row's slot is position 0 of its own first block
    assert list(feed.slot_mapping) == [0 * 8, 1 * 8, 2 * 8, 3 * 8]
    assert list(feed.active_mask) == [1, 1, 0, 0]
    assert list(feed.control) == [3, V - 1, V - 1, 33, 33, 0, 0, 1, 2, 0, 0]
    assert res.feed_calls == 1 and res.fetch_calls == 1 and res.model_calls == 3 and res.device_status == 0
    tokens = res.token_ids.reshape(B, 8)
    assert list(tokens[0, :3]) == [successor(5), successor(successor(5)), successor(successor(successor(5)))]
    assert list(tokens[1, :1]) == [successor(6)]
    assert (tokens[:, 3:] == -1).all() and (tokens[2:] == -1).all()
    assert list(res.executed) == [3, 3, 0, 0] and list(res.row_generations) == [1, 2, 0, 0]
    assert res.declared_input_bytes == 260 and res.declared_output_bytes == 368


def test_commit_state_constants():
    # native/resident_epoch_protocol.h:23-25
    assert (COMMIT_PREPARED, COMMIT_EXECUTING, COMMIT_COMMITTED) == (0, 1, 2)
