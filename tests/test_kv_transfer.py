"""KV transfer records and capture (cruise_amd.kv_transfer), on the CPU.

The behaviours the reference's tests/test_kv_transfer.py checks: the IPC
record carries only metadata in its fixed layout; exports are made once per
allocation with each cache's offset in it; a snapshot takes each imported
row's scheduler block into the row's slot.  Every validation rule is broken
once and named by the error; a damaged snapshot file is refused and a failed
write leaves no file behind.  The checksum is pinned against zlib.adler32 run
over the blocks the reference's loop selects (kv_transfer.py:159-174),
computed here by slicing a numpy view instead of by offsets, and against a
brute-force Adler-32 of the concatenated bytes.
"""
from __future__ import annotations

import os
import struct
import zlib
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import cruise_amd.kv_transfer as kvt
from cruise_amd.contract import CONTRACT_VERSION, ResidentEpochPlan, ResidentEpochRequest
from cruise_amd.kv_transfer import (
    BLOCK_ELEMENTS,
    ELEMENT_BYTES,
    GRAPH_BATCH_SIZE,
    HEADER,
    IPC_KEY_BYTES,
    IPC_KEY_COUNT,
    IPC_METADATA_BYTES,
    IPC_METADATA_HEADER,
    PAYLOAD_BYTES,
    TRANSFER_HEADER_BYTES,
    DeviceKVTransfer,
    TransferError,
    KVGeometry,
    ResidentKVSnapshot,
    capture_kv_device_transfer,
    capture_kv_snapshot,
    kv_payload_checksum,
    read_kv_snapshot,
    release_kv_device_exports,
    write_kv_snapshot,
)

SMALL = KVGeometry(layers=3, batch=4, block_size=4, kv_heads=2, head_size=8, element_bytes=2)


def importing(row, gen, block, pos=3):
    return ResidentEpochRequest(req_id=f"r{row}", row=row, generation=gen, token_id=42 + row, position=pos,
                                sequence_length=pos + 1, eos_token_id=151645, scheduler_block_ids=(block,),
                                device_block_ids=(2 * row, 2 * row + 1), state_owner="host", kv_import_required=True)


def plan_of(*reqs, steps=2):
    mask = [0] * 4
    for r in reqs:
        mask[r.row] = 1
    return ResidentEpochPlan(CONTRACT_VERSION, 4, steps, 8, tuple(reqs), tuple(mask))


def adler32_brute(data: bytes) -> int:
    a, b = 1, 0
    for byte in data:
        a = (a + byte) % 65521
        b = (b + a) % 65521
    return (b << 16) | a


def test_checksum_covers_k_then_v_layer_major_selected_rows():
    rng = np.random.default_rng(3)
    payload = rng.integers(0, 256, SMALL.payload_bytes, dtype=np.uint8)
    view = payload.reshape(2, SMALL.layers, SMALL.batch, SMALL.block_bytes)
    for mask in (0b0001, 0b0101, 0b1110, 0b1111):
        rows = [r for r in range(4) if mask >> r & 1]
        selected = b"".join(view[c, l, r].tobytes() for c in range(2) for l in range(SMALL.layers) for r in rows)
        expected = zlib.adler32(selected)
        assert kv_payload_checksum(payload.tobytes(), mask, SMALL) == expected
        assert expected == adler32_brute(selected)
    # a dropped row or a swapped K/V order changes it
    swapped = np.concatenate([view[1], view[0]]).tobytes()
    assert kv_payload_checksum(swapped, 0b0101, SMALL) != kv_payload_checksum(payload.tobytes(), 0b0101, SMALL)


def test_device_kv_transfer_wire_contract_contains_only_metadata():
    keys = tuple(bytes([i + 1]) * IPC_KEY_BYTES for i in range(IPC_KEY_COUNT))
    block = BLOCK_ELEMENTS * ELEMENT_BYTES
    t = DeviceKVTransfer(7, 0b0101, (11, 0, 13, 0), (2, 0, 5, 0), 8 * block, (0, block) * (IPC_KEY_COUNT // 2), keys)
    wire = t.wire_bytes()
    assert len(wire) == IPC_METADATA_BYTES == 4088
    assert IPC_METADATA_BYTES < PAYLOAD_BYTES // 1000
    fields = IPC_METADATA_HEADER.unpack_from(wire)
    assert fields[:4] == (kvt.IPC_METADATA_MAGIC, kvt.IPC_METADATA_VERSION, 0b0101, 8 * block)
    assert fields[4:8] == (11, 0, 13, 0) and fields[8:12] == (2, 0, 5, 0)
    assert fields[12:] == t.source_offsets
    assert wire[-IPC_KEY_BYTES:] == keys[-1]


def test_small_geometry_record_zero_pads_unused_layers():
    g = KVGeometry(layers=2, batch=4, block_size=4, kv_heads=1, head_size=8, element_bytes=4)
    keys = tuple(bytes([9]) * IPC_KEY_BYTES for _ in range(4))
    t = DeviceKVTransfer(5, 1, (3, 0, 0, 0), (1, 0, 0, 0), 10 * g.block_bytes, (0, 0, 2 * g.block_bytes, 0), keys, g)
    wire = t.wire_bytes()
    fields = IPC_METADATA_HEADER.unpack_from(wire)
    assert fields[12:16] == (0, 0, 2 * g.block_bytes, 0) and set(fields[16:]) == {0}
    assert wire[IPC_METADATA_HEADER.size + 4 * IPC_KEY_BYTES:] == bytes((IPC_KEY_COUNT - 4) * IPC_KEY_BYTES)


@pytest.mark.parametrize(
    ("change", "rule"),
    [
        ({"transfer_id": 0}, "transfer-id"),
        ({"import_mask": 0}, "mask-range"),
        ({"import_mask": 0b10000}, "mask-range"),
        ({"row_generations": (11, 0, 13)}, "generation-count"),
        ({"row_generations": (0, 0, 0, 0)}, "row-fields"),
        ({"block_ids": (2, 1, 5, 0)}, "row-fields"),
        ({"block_ids": (2, 0, 5)}, "block-count"),
        ({"source_bytes": 5 * BLOCK_ELEMENTS * ELEMENT_BYTES}, "block-range"),
        ({"source_bytes": 0}, "source-size"),
        ({"keys": (b"short",) * IPC_KEY_COUNT}, "key-format"),
        ({"keys": (bytes(IPC_KEY_BYTES),) * IPC_KEY_COUNT}, "key-format"),
        ({"keys": (b"\x01" * IPC_KEY_BYTES,)}, "key-count"),
        ({"source_offsets": (0,)}, "offset-count"),
    ],
)
def test_device_kv_transfer_validation(change, rule):
    block = BLOCK_ELEMENTS * ELEMENT_BYTES
    fields = dict(transfer_id=7, import_mask=0b0101, row_generations=(11, 0, 13, 0), block_ids=(2, 0, 5, 0),
                  source_bytes=8 * block, source_offsets=(0, block) * (IPC_KEY_COUNT // 2),
                  keys=tuple(b"\x01" * IPC_KEY_BYTES for _ in range(IPC_KEY_COUNT)))
    DeviceKVTransfer(**fields).validate()
    fields.update(change)
    with pytest.raises(TransferError) as raised:
        DeviceKVTransfer(**fields).validate()
    assert raised.value.rule == rule and isinstance(raised.value, ValueError)


def test_device_kv_export_uses_allocation_base_offsets(monkeypatch):
    exported = []
    view_bytes = 8 * BLOCK_ELEMENTS * ELEMENT_BYTES
    allocation = 2 * view_bytes + 2 * BLOCK_ELEMENTS * ELEMENT_BYTES

    class FakeTensor:
        is_cuda = True

        def __init__(self, ptr):
            self.ptr = ptr

        def is_contiguous(self):
            return True

        def data_ptr(self):
            return self.ptr

        def numel(self):
            return view_bytes // ELEMENT_BYTES

        def element_size(self):
            return ELEMENT_BYTES

        def dim(self):
            return 4

        shape = (8, 128, 4, 128)

    caches, bases = [], {}
    for layer in range(28):
        base = 0x1000000 + layer * 0x4000000
        key, value = FakeTensor(base), FakeTensor(base + view_bytes)
        bases[key.ptr] = bases[value.ptr] = base
        caches.append((key, value))
    monkeypatch.setattr(kvt, "_REGISTRY", kvt._ExportRegistry())
    monkeypatch.setattr(kvt, "_allocation_of", lambda ptr: (bases[ptr], allocation))
    monkeypatch.setattr(kvt, "_ipc_handle", lambda base: exported.append(base) or base.to_bytes(8, "little") * 8)
    worker = SimpleNamespace(model_runner=SimpleNamespace(kv_caches=caches))
    plan = plan_of(importing(0, 7, 0))
    transfer = capture_kv_device_transfer(worker, plan)
    assert len(exported) == IPC_KEY_COUNT // 2  # one export per allocation
    assert transfer.source_bytes == allocation
    assert transfer.source_offsets == (0, view_bytes) * (IPC_KEY_COUNT // 2)
    assert all(transfer.keys[i] == transfer.keys[i + 1] for i in range(0, IPC_KEY_COUNT, 2))
    assert transfer.row_generations == (7, 0, 0, 0) and transfer.block_ids == (0, 0, 0, 0)
    # the exports are reused while the caches stay where they are
    capture_kv_device_transfer(worker, plan)
    assert len(exported) == IPC_KEY_COUNT // 2
    release_kv_device_exports(worker)
    capture_kv_device_transfer(worker, plan)
    assert len(exported) == IPC_KEY_COUNT


def test_device_kv_export_rejects_unequal_allocations(monkeypatch):
    class T:
        is_cuda = True
        shape = (8, 128, 4, 128)

        def __init__(self, p):
            self.p = p

        def is_contiguous(self):
            return True

        def data_ptr(self):
            return self.p

        def numel(self):
            return 16

        def element_size(self):
            return 2

        def dim(self):
            return 4

    monkeypatch.setattr(kvt, "_allocation_of", lambda ptr: (ptr, 1 << 20 if ptr < 100 else 2 << 20))
    worker = SimpleNamespace(model_runner=SimpleNamespace(kv_caches=[(T(1), T(2)), (T(200), T(300))]))
    monkeypatch.setattr(kvt, "_REGISTRY", kvt._ExportRegistry())
    with pytest.raises(RuntimeError, match="differ in size"):
        capture_kv_device_transfer(worker, plan_of(importing(0, 7, 0)))


def test_capture_stock_paged_kv_uses_scheduler_block_and_resident_row():
    key = torch.zeros((2, 128, 4, 128), dtype=torch.bfloat16)
    value = torch.zeros_like(key)
    key[1].fill_(1)
    value[1].fill_(2)
    worker = SimpleNamespace(model_runner=SimpleNamespace(kv_caches=[(key, value)] * 28))
    snap = capture_kv_snapshot(worker, plan_of(importing(1, 7, 1)))
    assert HEADER.size == TRANSFER_HEADER_BYTES == 80
    assert len(snap.payload) == PAYLOAD_BYTES
    assert snap.import_mask == 0b0010 and snap.row_generations == (0, 7, 0, 0)
    assert snap.checksum == kv_payload_checksum(snap.payload, 0b0010)
    row_bytes = BLOCK_ELEMENTS * ELEMENT_BYTES
    value_base = 28 * GRAPH_BATCH_SIZE * row_bytes
    assert struct.unpack_from("<H", snap.payload, row_bytes)[0] == 0x3F80  # bf16 1.0 in row 1's K slot
    assert struct.unpack_from("<H", snap.payload, value_base + row_bytes)[0] == 0x4000  # bf16 2.0 in its V slot
    assert struct.unpack_from("<H", snap.payload, 0)[0] == 0


def test_capture_stock_paged_kv_imports_multiple_scheduler_blocks_by_row():
    key = torch.zeros((4, 128, 4, 128), dtype=torch.bfloat16)
    value = torch.zeros_like(key)
    for b in range(4):
        key[b].fill_(b + 1)
        value[b].fill_(b + 5)
    worker = SimpleNamespace(model_runner=SimpleNamespace(kv_caches=[(key, value)] * 28))
    snap = capture_kv_snapshot(worker, plan_of(importing(0, 10, 2), importing(2, 12, 0), importing(3, 13, 3), steps=1))
    assert snap.import_mask == 0b1101 and snap.row_generations == (10, 0, 12, 13)
    row_bytes = BLOCK_ELEMENTS * ELEMENT_BYTES
    for row, word in {0: 0x4040, 1: 0, 2: 0x3F80, 3: 0x4080}.items():
        assert struct.unpack_from("<H", snap.payload, row * row_bytes)[0] == word


def test_snapshot_file_round_trip_and_header(tmp_path):
    if not os.path.isdir("/dev/shm"):
        pytest.skip("no /dev/shm")
    rng = np.random.default_rng(9)
    payload = rng.integers(0, 256, SMALL.payload_bytes, dtype=np.uint8).tobytes()
    snap = ResidentKVSnapshot(123456789, 0b1001, (4, 0, 0, 6), payload, kv_payload_checksum(payload, 0b1001, SMALL), SMALL)
    path = f"/dev/shm/cruise-kvt-test-{os.getpid()}"
    try:
        write_kv_snapshot(path, snap)
        raw = open(path, "rb").read()
        fields = HEADER.unpack_from(raw)
        assert fields[:6] == (kvt.TRANSFER_MAGIC, 1, 80, 123456789, SMALL.payload_bytes, 0b1001)
        assert fields[6:10] == (4, 0, 0, 6)
        assert fields[10:16] == (3, 4, 4, 2, 8, 2) and fields[16] == snap.checksum
        assert raw[80:] == payload
        assert read_kv_snapshot(path) == snap
    finally:
        os.unlink(path)
    with pytest.raises(TransferError) as raised:
        write_kv_snapshot(tmp_path / "x", snap)
    assert raised.value.rule == "location"


@pytest.mark.parametrize(
    ("change", "rule"),
    [
        ({"transfer_id": 0}, "transfer-id"),
        ({"import_mask": 0b10000}, "mask-range"),
        ({"row_generations": (4, 1, 0, 6)}, "generation-selects-row"),
        ({"row_generations": (4, 0, 0, -6)}, "generation-sign"),
        ({"payload": b"x"}, "payload-size"),
        ({"checksum": 1}, "checksum"),
    ],
)
def test_snapshot_validation(change, rule):
    payload = bytes(SMALL.payload_bytes)
    fields = dict(transfer_id=1, import_mask=0b1001, row_generations=(4, 0, 0, 6), payload=payload,
                  checksum=kv_payload_checksum(payload, 0b1001, SMALL), geometry=SMALL)
    ResidentKVSnapshot(**fields).validate()
    fields.update(change)
    with pytest.raises(TransferError) as raised:
        ResidentKVSnapshot(**fields).validate()
    assert raised.value.rule == rule


def test_snapshot_file_rejects_a_damaged_header_or_size():
    if not os.path.isdir("/dev/shm"):
        pytest.skip("no /dev/shm")
    payload = bytes(range(256)) * (SMALL.payload_bytes // 256)
    snap = ResidentKVSnapshot(9, 0b0010, (0, 3, 0, 0), payload, kv_payload_checksum(payload, 0b0010, SMALL), SMALL)
    raw = snap.header() + payload
    assert ResidentKVSnapshot.parse(raw) == snap
    for damaged, rule in ((raw[:40], "file-size"), (raw[:-1], "file-size"), (b"\0" + raw[1:], "magic")):
        with pytest.raises(TransferError) as raised:
            ResidentKVSnapshot.parse(damaged)
        assert raised.value.rule == rule
    flipped = bytearray(raw)
    flipped[TRANSFER_HEADER_BYTES + 5 * SMALL.block_bytes] ^= 1  # row 1's K block of layer 1
    with pytest.raises(TransferError, match="checksum"):
        ResidentKVSnapshot.parse(bytes(flipped))


def test_snapshot_writer_leaves_no_partial_file_on_failure(monkeypatch):
    if not os.path.isdir("/dev/shm"):
        pytest.skip("no /dev/shm")
    payload = bytes(SMALL.payload_bytes)
    snap = ResidentKVSnapshot(5, 0b0001, (2, 0, 0, 0), payload, kv_payload_checksum(payload, 1, SMALL), SMALL)
    folder = f"/dev/shm/cruise-kvt-fail-{os.getpid()}"
    os.makedirs(folder, exist_ok=True)
    try:
        def boom(fd):
            raise OSError("disk gone")

        monkeypatch.setattr(kvt.os, "fsync", boom)
        with pytest.raises(OSError, match="disk gone"):
            write_kv_snapshot(f"{folder}/snap", snap)
        assert os.listdir(folder) == []
    finally:
        for name in os.listdir(folder):
            os.unlink(os.path.join(folder, name))
        os.rmdir(folder)
