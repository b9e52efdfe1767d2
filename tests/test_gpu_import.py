"""GPU parity of the KV-import epoch on the tiny fp32 model (CTRL:387-446).

An import epoch carries a payload of one block per layer per row ([K|V]
[layers][B][block], kv_transfer.py:31) ahead of the feed.  The device copies
the blocks of the masked rows into each row's first block, adopts the rows as
resident, checksums the imported blocks (Adler-32, key then value cache,
layer-major, rows ascending) and runs the epoch.  Checked against the oracle
controller (history and control record bit-exact, caches at tolerance) and
the checksum against a restatement of the reference's host
``kv_payload_checksum`` (kv_transfer.py:159-174).  The bridge path reads the
payload from a transfer file (80-byte header, BRIDGE:72-154) and returns 34
on a checksum mismatch, 13 on a bad file.
"""
from __future__ import annotations

import os
import struct
import tempfile
import zlib

import numpy as np
import pytest
import torch

from cruise_amd.runtime import pack_feed, tiling_bytes
from oracle.controller import IMPORT_GRAPH_FLAG, EpochFeed, control_input_elements
from oracle.weights import generate_weights
from oracle.workloads import C1, identity_table, slot_of
from parity import TeacherForcing, assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C1
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
L = W.dims.num_layers
KVH = W.dims.num_kv_heads
D = W.dims.head_dim
BLOCK_ELEMS = BS * KVH * D
TRANSFER_MAGIC = 0x4352554953454B56
HEADER = struct.Struct("<QIIQQI4i7I")  # kv_transfer.py:31


@pytest.fixture(scope="module")
def weights():
    return generate_weights(W.dims, W.seed)


@pytest.fixture(scope="module")
def rt(weights):
    r = make_runtime(W, weights)
    yield r
    r.close()


def reset(rt):
    zeros = torch.zeros(rt.cache_bytes // 4, dtype=torch.float32, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))


def make_payload(seed: int) -> bytes:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(2 * L * B * BLOCK_ELEMS, generator=g) * 0.25).numpy().astype(np.float32).tobytes()


def payload_checksum(payload: bytes, mask: int) -> int:
    """kv_transfer.py:159-174 restated: zlib.adler32 chained over the blocks."""
    block_bytes = BLOCK_ELEMS * 4
    cache_bytes = L * B * block_bytes
    checksum = 1
    for base in (0, cache_bytes):
        for layer in range(L):
            for row in range(B):
                if mask & (1 << row):
                    off = base + (layer * B + row) * block_bytes
                    checksum = zlib.adler32(payload[off : off + block_bytes], checksum)
    return checksum & 0xFFFFFFFF


def import_case(rt, weights, *, mask, tokens, positions, lengths, active, gens, K, payload):
    table = identity_table(B, BPR)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[2 + B] = IMPORT_GRAPH_FLAG | mask
    control[3 + B :] = gens
    tokens = np.asarray(tokens, dtype=np.int64)
    positions = np.asarray(positions, dtype=np.int64)
    lengths = np.asarray(lengths, dtype=np.int32)
    active = np.asarray(active, dtype=np.int32)
    reset(rt)
    hist, ctrl = rt.proc(pack_feed(tokens, positions, lengths, None, active, table, tiling_bytes(), control, payload=payload))
    _, ctl = oracle_controller(W, weights)
    ctl.token_override = TeacherForcing(hist, rel_tol(W.dims))
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control, import_payload=payload))
    return hist, ctrl, ref, ctl


def test_import_epoch_matches_oracle(rt, weights):
    payload = make_payload(11)
    mask = 0b0101  # rows 0 and 2 import a 3- and 5-token prefix; row 1 starts fresh; row 3 is empty
    hist, ctrl, ref, ctl = import_case(
        rt, weights, mask=mask, tokens=[17, 42, 99, 0], positions=[3, 0, 5, 0], lengths=[4, 1, 6, 0],
        active=[1, 1, 1, 0], gens=[7, 8, 9, 0], K=3, payload=payload,
    )
    assert not ctl.token_override.mismatches, ctl.token_override.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    assert ctrl[3] == 0 and ctrl[4] == 3
    assert int(np.uint32(np.int32(ctrl[5]))) == payload_checksum(payload, mask)
    key = torch.zeros(rt.cache_bytes // 4, dtype=torch.float32)
    rt.read_state("key_cache", key)
    key = key.view_as(ctl.resident_key)
    assert_close_rel(key, ctl.resident_key, rel_tol(W.dims), "resident keys after import")
    src = torch.frombuffer(bytearray(payload), dtype=torch.float32).view(2, L, B, BS, KVH, D)
    # the imported prefix (positions before the row's first step) is the payload, bit for bit
    assert torch.equal(key[:, 0, :3], src[0, :, 0, :3])
    assert torch.equal(key[:, 4, :5], src[0, :, 2, :5])
    rows = rt.resident_rows()
    assert list(rows[0]) == [7, 8, 9, 0] and list(rows[2][:3]) == [6, 3, 8]  # gens; positions after 3 steps


def test_import_then_continuity_fallback(rt, weights):
    """Row 1 continues a generation it never had: 212 after the import ran,
    so the checksum is still emitted and the imported rows stay adopted."""
    payload = make_payload(12)
    mask = 0b0001
    hist, ctrl, ref, ctl = import_case(
        rt, weights, mask=mask, tokens=[17, 42, 0, 0], positions=[3, 2, 0, 0], lengths=[4, 3, 0, 0],
        active=[1, 1, 0, 0], gens=[7, 8, 0, 0], K=2, payload=payload,
    )
    assert ctrl[3] == 212 and ref.control[3] == 212
    np.testing.assert_array_equal(ctrl, ref.control)
    assert int(np.uint32(np.int32(ctrl[5]))) == payload_checksum(payload, mask)
    rows = rt.resident_rows()
    assert rows[0][0] == 7 and rows[2][0] == 3 and rows[4][0] == 1  # row 0 adopted at position 3


def test_partial_import_then_invalid_row(rt, weights):
    """Mask 0b0011 with row 1 inactive: CTRL:402-428 copies row 0's block and
    adopts it, then rejects row 1 (201) before the checksum.  Row 0's KV and
    resident record must be the oracle's: adopted, block copied bit for bit,
    the other blocks of the row cleared."""
    payload = make_payload(14)
    mask = 0b0011
    hist, ctrl, ref, ctl = import_case(
        rt, weights, mask=mask, tokens=[17, 42, 0, 0], positions=[3, 0, 0, 0], lengths=[4, 1, 0, 0],
        active=[1, 0, 0, 0], gens=[7, 0, 0, 0], K=2, payload=payload,
    )
    assert ctrl[3] == 201 and ref.control[3] == 201
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    assert ctrl[5] == 0  # the import stopped before its checksum
    rows = rt.resident_rows()
    np.testing.assert_array_equal(rows[0], ctl.resident_generation)
    np.testing.assert_array_equal(rows[1], ctl.resident_token)
    np.testing.assert_array_equal(rows[2], ctl.resident_position)
    np.testing.assert_array_equal(rows[3], ctl.resident_length)
    np.testing.assert_array_equal(rows[4], ctl.resident_valid)
    assert rows[0][0] == 7 and rows[4][0] == 1
    for name, ref_cache in (("key_cache", ctl.resident_key), ("value_cache", ctl.resident_value)):
        got = torch.zeros(rt.cache_bytes // 4, dtype=torch.float32)
        rt.read_state(name, got)
        assert torch.equal(got.view_as(ref_cache), ref_cache), f"{name} after a partial import"


def write_transfer(path: str, transfer_id: int, mask: int, gens, payload: bytes, checksum: int) -> None:
    header = HEADER.pack(TRANSFER_MAGIC, 1, HEADER.size, transfer_id, len(payload), mask, *gens, L, B, BS, KVH, D, 4, checksum)
    assert len(header) == 80
    with open(path, "wb") as f:
        f.write(header)
        f.write(payload)


def test_bridge_transfer_import(rt, weights):
    payload = make_payload(13)
    mask = 0b0010
    gens = [0, 5, 0, 0]
    fd, path = tempfile.mkstemp(prefix="cruise-kv-", dir="/dev/shm")
    os.close(fd)
    try:
        write_transfer(path, 99, mask, gens, payload, payload_checksum(payload, mask))
        reset(rt)
        out = rt.execute(1, 2, [0, 31, 0, 0], [0, 4, 0, 0], [0, 5, 0, 0], [W.eos] * B, gens, transfer_path=path, transfer_id=99)
        assert out.status == 0 and out.device_status == 0, (out.status, out.device_status)
        assert out.kv_import_checksum == payload_checksum(payload, mask)
        assert out.commit_state == 2 and list(out.executed) == [0, 2, 0, 0]
        # the first generated token follows the imported prefix: compare with the oracle
        _, ctl = oracle_controller(W, weights)
        table = identity_table(B, BPR)
        control = np.zeros(control_input_elements(B), dtype=np.int32)
        control[0] = 2
        control[1 : 1 + B] = W.eos
        control[2 + B] = IMPORT_GRAPH_FLAG | mask
        control[3 + B :] = gens
        ctl.token_override = TeacherForcing(out.token_ids.T.copy(), rel_tol(W.dims))
        ref = ctl.proc(EpochFeed(np.array([0, 31, 0, 0]), np.array([0, 4, 0, 0]), np.array([0, 5, 0, 0], dtype=np.int32),
                                 np.zeros(B, dtype=np.int32), np.array([0, 1, 0, 0], dtype=np.int32), table.reshape(-1),
                                 tiling_bytes(), control, import_payload=payload))
        assert not ctl.token_override.mismatches, ctl.token_override.mismatches
        assert list(out.token_ids[1, :2]) == list(ref.history[:2, 1])
        # a wrong checksum in the header: the device checksum disagrees -> 34
        write_transfer(path, 100, mask, gens, payload, payload_checksum(payload, mask) ^ 1)
        reset(rt)
        out = rt.execute(1, 2, [0, 31, 0, 0], [0, 4, 0, 0], [0, 5, 0, 0], [W.eos] * B, gens, transfer_path=path, transfer_id=100)
        assert out.status == 34
        # a transfer id that does not match the file -> 13
        out = rt.execute(1, 2, [0, 31, 0, 0], [0, 4, 0, 0], [0, 5, 0, 0], [W.eos] * B, gens, transfer_path=path, transfer_id=101)
        assert out.status == 13
    finally:
        os.unlink(path)
