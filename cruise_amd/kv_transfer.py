"""Paged-KV transfer into the resident epoch: host snapshot files and
device-to-device transfer through HIP IPC.

Mirrors src/vllm_ascend_resident_epoch/kv_transfer.py.  A prefilled row
enters device ownership by importing one KV block per layer (its first
block, positions 0..block_size-1) from the stock cache the prompt was
prefilled into:

* host snapshot: the blocks are gathered into one payload
  ``[K|V][layer][row][block_size, kv_heads, head]`` and written to a file
  under /dev/shm with an 80-byte header (kv_transfer.py:31, 431-466); the
  engine reads it, imports it with the epoch's one feed copy and proves the
  import with an Adler-32 of the imported bytes (kv_transfer.py:159-174).
* device IPC: only metadata crosses the process boundary (4,088 bytes,
  kv_transfer.py:33-34, 67-137): for each of the 2 x layers caches an IPC
  handle of the allocation holding it and the cache's offset inside it, plus
  the scheduler block of every imported row.  The engine opens the handles
  once and copies the blocks device to device.

The one difference from the reference is the key: an Ascend IPC key is an
ASCII name, a HIP IPC handle is a 64-byte binary record
(``hipIpcMemHandle_t``), so ``DeviceKVTransfer.keys`` holds 64-byte
``bytes`` values, written to the same 64-byte slots of the record.
"""
from __future__ import annotations

import ctypes
import os
import secrets
import struct
import zlib
from dataclasses import dataclass, field
from functools import lru_cache
from pathlib import Path
from typing import Any

TRANSFER_MAGIC = 0x4352554953454B56  # "CRUISEKV"
TRANSFER_VERSION = 1
TRANSFER_HEADER_BYTES = 80
IPC_METADATA_MAGIC = 0x4352554953454950  # "CRUISEIP"
IPC_METADATA_VERSION = 2
IPC_KEY_BYTES = 64  # also sizeof(hipIpcMemHandle_t)


@dataclass(frozen=True)
class KVGeometry:
    """Shape of the imported blocks (Qwen2.5-7B at B=4 by default)."""

    layers: int = 28
    batch: int = 4
    block_size: int = 128
    kv_heads: int = 4
    head_size: int = 128
    element_bytes: int = 2

    @property
    def block_elements(self) -> int:
        return self.block_size * self.kv_heads * self.head_size

    @property
    def block_bytes(self) -> int:
        return self.block_elements * self.element_bytes

    @property
    def cache_bytes(self) -> int:
        """Bytes of one cache (K or V) of the payload."""
        return self.layers * self.batch * self.block_bytes

    @property
    def payload_bytes(self) -> int:
        return 2 * self.cache_bytes

    @property
    def key_count(self) -> int:
        return 2 * self.layers


QWEN7B_B4 = KVGeometry()

LAYERS = QWEN7B_B4.layers
GRAPH_BATCH_SIZE = QWEN7B_B4.batch
BLOCK_SIZE = QWEN7B_B4.block_size
NUM_KV_HEADS = QWEN7B_B4.kv_heads
HEAD_SIZE = QWEN7B_B4.head_size
ELEMENT_BYTES = QWEN7B_B4.element_bytes
BLOCK_ELEMENTS = QWEN7B_B4.block_elements
ROW_BYTES = 2 * QWEN7B_B4.block_bytes
PAYLOAD_BYTES = QWEN7B_B4.payload_bytes
IPC_KEY_COUNT = QWEN7B_B4.key_count

# Little-endian records: the snapshot header and the IPC metadata header
# (kv_transfer.py:31, 33).
HEADER = struct.Struct("<QIIQQI4i7I")
IPC_METADATA_HEADER = struct.Struct(f"<QIIQ4i4i{IPC_KEY_COUNT}Q")
IPC_METADATA_BYTES = IPC_METADATA_HEADER.size + IPC_KEY_COUNT * IPC_KEY_BYTES
assert HEADER.size == TRANSFER_HEADER_BYTES and IPC_METADATA_BYTES == 4088


def _check(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _check_mask_and_generations(mask: int, generations: tuple[int, ...], rows: int, what: str) -> None:
    _check(len(generations) == rows, f"{what} generation vector must have {rows} rows")
    _check(0 < mask < 1 << rows, f"{what} mask must select at least one row")


def kv_payload_checksum(payload: bytes, import_mask: int, geometry: KVGeometry = QWEN7B_B4) -> int:
    """Adler-32 over the imported blocks: the K cache, then the V cache, each
    layer-major and, inside a layer, in ascending row order over the rows of
    import_mask (kv_transfer.py:159-174; the engine's device checksum sums
    the same bytes)."""
    g = geometry
    _check(len(payload) == g.payload_bytes, "cannot checksum an incomplete KV transfer payload")
    view = memoryview(payload)
    value = 1
    rows = [r for r in range(g.batch) if import_mask & (1 << r)]
    for cache in range(2):
        for layer in range(g.layers):
            for row in rows:
                start = cache * g.cache_bytes + (layer * g.batch + row) * g.block_bytes
                value = zlib.adler32(view[start : start + g.block_bytes], value)
    return value & 0xFFFFFFFF


@dataclass(frozen=True)
class ResidentKVSnapshot:
    """A host copy of the imported blocks (kv_transfer.py:37-64)."""

    transfer_id: int
    import_mask: int
    row_generations: tuple[int, ...]
    payload: bytes
    checksum: int
    geometry: KVGeometry = field(default=QWEN7B_B4)

    def validate(self) -> None:
        g = self.geometry
        _check(self.transfer_id > 0, "KV transfer id must be positive")
        _check_mask_and_generations(self.import_mask, tuple(self.row_generations), g.batch, "KV transfer")
        _check(all(gen >= 0 for gen in self.row_generations), "KV transfer generations must be non-negative")
        for row, gen in enumerate(self.row_generations):
            _check(bool(self.import_mask & (1 << row)) == (gen > 0), "KV transfer mask and generations disagree")
        _check(
            len(self.payload) == g.payload_bytes,
            f"KV transfer payload must be {g.payload_bytes} bytes, got {len(self.payload)}",
        )
        _check(
            self.checksum == kv_payload_checksum(self.payload, self.import_mask, g),
            "KV transfer checksum does not match its payload",
        )


@dataclass(frozen=True)
class DeviceKVTransfer:
    """IPC metadata of a device-to-device import (kv_transfer.py:67-137).

    keys[2*l] / keys[2*l+1]: the HIP IPC handle (64 bytes) of the allocation
    holding layer l's K / V cache; source_offsets: each cache's byte offset
    in its allocation; source_bytes: the common allocation size; block_ids:
    the scheduler block of each imported row (0 for the others)."""

    transfer_id: int
    import_mask: int
    row_generations: tuple[int, ...]
    block_ids: tuple[int, ...]
    source_bytes: int
    source_offsets: tuple[int, ...]
    keys: tuple[bytes, ...]
    geometry: KVGeometry = field(default=QWEN7B_B4)

    def validate(self) -> None:
        g = self.geometry
        _check(g.key_count <= IPC_KEY_COUNT, "device KV transfer has more caches than the wire record")
        _check(self.transfer_id > 0, "device KV transfer id must be positive")
        _check(len(self.block_ids) == g.batch, f"device KV transfer block vector must have {g.batch} rows")
        _check_mask_and_generations(self.import_mask, tuple(self.row_generations), g.batch, "device KV transfer")
        _check(self.source_bytes > 0, "device KV transfer source size must be positive")
        _check(len(self.source_offsets) == g.key_count, f"device KV transfer must carry {g.key_count} source offsets")
        _check(len(self.keys) == g.key_count, f"device KV transfer must carry {g.key_count} keys")
        for row in range(g.batch):
            gen, block = self.row_generations[row], self.block_ids[row]
            if self.import_mask & (1 << row):
                _check(gen > 0 and block >= 0, "selected device KV rows need generation and block")
                end = (block + 1) * g.block_bytes
                for offset in self.source_offsets:
                    _check(0 <= offset and offset + end <= self.source_bytes, "device KV block is outside its exported allocation")
            else:
                _check(gen == 0 and block == 0, "unselected device KV rows must be zeroed")
        for key in self.keys:
            _check(
                isinstance(key, (bytes, bytearray)) and len(key) == IPC_KEY_BYTES and any(key),
                "device KV IPC key does not fit the wire contract",
            )

    def wire_bytes(self) -> bytes:
        """The 4,088-byte record the engine reads (ResidentEpochIpcMetadata);
        slots of layers past geometry.layers stay zero."""
        self.validate()
        pad = IPC_KEY_COUNT - len(self.keys)
        header = IPC_METADATA_HEADER.pack(
            IPC_METADATA_MAGIC,
            IPC_METADATA_VERSION,
            self.import_mask,
            self.source_bytes,
            *self.row_generations,
            *self.block_ids,
            *self.source_offsets,
            *([0] * pad),
        )
        record = header + b"".join(bytes(k) for k in self.keys) + bytes(pad * IPC_KEY_BYTES)
        assert len(record) == IPC_METADATA_BYTES
        return record


# ---------------------------------------------------------------------------
# Host snapshot files
# ---------------------------------------------------------------------------
def write_kv_snapshot(path: str | Path, snapshot: ResidentKVSnapshot) -> None:
    """Write header + payload atomically (temporary file, fsync, rename);
    the file must lie under /dev/shm (kv_transfer.py:431-466)."""
    snapshot.validate()
    g = snapshot.geometry
    target = Path(path).resolve()
    _check(str(target).startswith("/dev/shm/"), "KV transfer files must be under /dev/shm")
    target.parent.mkdir(parents=True, exist_ok=True)
    staging = target.with_name(f".{target.name}.tmp-{os.getpid()}-{snapshot.transfer_id}")
    if staging.exists():
        raise RuntimeError(f"stale KV transfer temporary file exists: {staging}")
    header = HEADER.pack(
        TRANSFER_MAGIC,
        TRANSFER_VERSION,
        TRANSFER_HEADER_BYTES,
        snapshot.transfer_id,
        len(snapshot.payload),
        snapshot.import_mask,
        *snapshot.row_generations,
        g.layers,
        g.batch,
        g.block_size,
        g.kv_heads,
        g.head_size,
        g.element_bytes,
        snapshot.checksum,
    )
    try:
        with staging.open("xb") as out:
            out.write(header)
            out.write(snapshot.payload)
            out.flush()
            os.fsync(out.fileno())
        os.replace(staging, target)
    finally:
        staging.unlink(missing_ok=True)


def read_kv_snapshot(path: str | Path) -> ResidentKVSnapshot:
    """Parse a snapshot file back (header checks as the engine makes them)."""
    raw = Path(path).read_bytes()
    _check(len(raw) >= TRANSFER_HEADER_BYTES, "KV transfer file is shorter than its header")
    fields = HEADER.unpack_from(raw)
    magic, version, header_bytes, transfer_id, payload_bytes, mask = fields[:6]
    gens = tuple(fields[6:10])
    layers, batch, block_size, kv_heads, head_size, element_bytes, checksum = fields[10:]
    _check(magic == TRANSFER_MAGIC and version == TRANSFER_VERSION, "not a KV transfer file")
    _check(header_bytes == TRANSFER_HEADER_BYTES, "KV transfer header size mismatch")
    _check(len(raw) == header_bytes + payload_bytes, "KV transfer file size mismatch")
    g = KVGeometry(layers, batch, block_size, kv_heads, head_size, element_bytes)
    snap = ResidentKVSnapshot(transfer_id, mask, gens, raw[header_bytes:], checksum, g)
    snap.validate()
    return snap


# ---------------------------------------------------------------------------
# Capture from the stock KV cache of a worker
# ---------------------------------------------------------------------------
def _stock_caches(worker: Any) -> list:
    runner = getattr(worker, "model_runner", None)
    caches = getattr(runner, "kv_caches", None)
    if not isinstance(caches, list) or not caches:
        raise RuntimeError("stock KV cache layout is not a list of per-layer K/V pairs")
    for layer in caches:
        if not isinstance(layer, (tuple, list)) or len(layer) < 2:
            raise RuntimeError("stock vLLM KV cache layer is not a K/V pair")
    return caches


def _geometry_of(caches: list, batch: int) -> KVGeometry:
    """Geometry of stock caches laid out [blocks, block_size, kv_heads, head]."""
    key = caches[0][0]
    if key.dim() != 4:
        raise RuntimeError("stock KV cache entries must be [blocks, block_size, kv_heads, head]")
    _, bs, kvh, hd = (int(s) for s in key.shape)
    return KVGeometry(len(caches), batch, bs, kvh, hd, int(key.element_size()))


def _import_rows(plan: Any, what: str) -> list:
    rows = [r for r in plan.requests if r.kv_import_required]
    if not rows:
        raise ValueError(f"{what} requested for a plan without imports")
    for r in rows:
        if len(r.scheduler_block_ids) != 1:
            raise ValueError(f"{what} requires one scheduler block per row")
    return rows


def capture_kv_snapshot(worker: Any, plan: Any, batch: int | None = None) -> ResidentKVSnapshot:
    """Copy each imported row's scheduler block of every layer into a
    compact payload (kv_transfer.py:362-428)."""
    import torch

    rows = _import_rows(plan, "KV snapshot")
    caches = _stock_caches(worker)
    g = _geometry_of(caches, batch or plan.graph_batch_size)
    if plan.logical_capacity > g.block_size:
        raise ValueError("a snapshot transfers one block per row: capacity must fit one block")
    block_of = {r.row: int(r.scheduler_block_ids[0]) for r in rows}
    parts: list[list] = [[], []]
    for key, value in (layer[:2] for layer in caches):
        for cache, tensor in ((0, key), (1, value)):
            if tensor.dtype != key.dtype:
                raise ValueError("K and V caches differ in dtype")
            for row in range(g.batch):
                block = block_of.get(row)
                if block is None:
                    parts[cache].append(torch.zeros(tensor.shape[1:], dtype=tensor.dtype))
                    continue
                if not 0 <= block < tensor.shape[0]:
                    raise ValueError("scheduler block is outside the stock KV cache")
                parts[cache].append(tensor[block].detach().to("cpu").contiguous())
    payload = b"".join(
        torch.stack(p).contiguous().view(torch.uint8).numpy().tobytes() for p in parts
    )
    gens = [0] * g.batch
    for r in rows:
        gens[r.row] = int(r.generation)
    mask = sum(1 << r.row for r in rows)
    snap = ResidentKVSnapshot(secrets.randbits(63) or 1, mask, tuple(gens), payload,
                              kv_payload_checksum(payload, mask, g), g)
    snap.validate()
    return snap


# HIP runtime entry points used by the exporting side.
@lru_cache(maxsize=1)
def _hip() -> ctypes.CDLL:
    lib = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
    lib.hipMemGetAddressRange.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p]
    lib.hipMemGetAddressRange.restype = ctypes.c_int
    lib.hipIpcGetMemHandle.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.hipIpcGetMemHandle.restype = ctypes.c_int
    return lib


def _allocation_of(data_ptr: int) -> tuple[int, int]:
    """(base, size) of the device allocation containing data_ptr."""
    base, size = ctypes.c_void_p(), ctypes.c_size_t()
    rc = _hip().hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), ctypes.c_void_p(data_ptr))
    if rc != 0 or not base.value or size.value == 0:
        raise RuntimeError(f"cannot resolve the device allocation holding the stock KV cache (hip error {rc})")
    return int(base.value), int(size.value)


def _ipc_handle(base: int) -> bytes:
    handle = ctypes.create_string_buffer(IPC_KEY_BYTES)
    rc = _hip().hipIpcGetMemHandle(handle, ctypes.c_void_p(base))
    if rc != 0:
        raise RuntimeError(f"hipIpcGetMemHandle failed for a stock KV allocation (hip error {rc})")
    return handle.raw


@dataclass
class _DeviceKVExportTable:
    signature: tuple[tuple[int, int, int], ...]  # (data_ptr, allocation base, allocation size) per cache
    source_bytes: int
    source_offsets: tuple[int, ...]
    keys: tuple[bytes, ...]


def _device_exports(worker: Any, caches: list) -> _DeviceKVExportTable:
    """Export every allocation holding a stock cache once per worker
    lifetime (kv_transfer.py:266-319): a HIP IPC handle stays valid while
    the allocation lives, so it is reused until the caches move."""
    entries = []
    for layer in caches:
        for tensor in layer[:2]:
            if not getattr(tensor, "is_cuda", False) or not tensor.is_contiguous():
                raise RuntimeError("stock KV cache entries must be contiguous device tensors for IPC export")
            ptr = int(tensor.data_ptr())
            base, size = _allocation_of(ptr)
            if ptr + tensor.numel() * tensor.element_size() > base + size:
                raise RuntimeError("stock KV cache entry extends past its device allocation")
            entries.append((ptr, base, size))
    sizes = {size for _, _, size in entries}
    if len(sizes) != 1:
        raise RuntimeError("key/value KV allocations do not have a common size")
    signature = tuple(entries)
    current = getattr(worker, "_resident_epoch_device_kv_exports", None)
    if isinstance(current, _DeviceKVExportTable) and current.signature == signature:
        return current
    handles: dict[int, bytes] = {}
    for _, base, _ in entries:
        if base not in handles:
            handles[base] = _ipc_handle(base)
    table = _DeviceKVExportTable(
        signature=signature,
        source_bytes=sizes.pop(),
        source_offsets=tuple(ptr - base for ptr, base, _ in entries),
        keys=tuple(handles[base] for _, base, _ in entries),
    )
    worker._resident_epoch_device_kv_exports = table
    return table


def capture_kv_device_transfer(worker: Any, plan: Any, batch: int | None = None) -> DeviceKVTransfer:
    """IPC metadata for importing the plan's rows, every KV byte staying on
    the device (kv_transfer.py:322-352)."""
    rows = _import_rows(plan, "device KV transfer")
    caches = _stock_caches(worker)
    g = _geometry_of(caches, batch or plan.graph_batch_size)
    table = _device_exports(worker, caches)
    blocks = [0] * g.batch
    gens = [0] * g.batch
    for r in rows:
        blocks[r.row] = int(r.scheduler_block_ids[0])
        gens[r.row] = int(r.generation)
    transfer = DeviceKVTransfer(
        transfer_id=secrets.randbits(63) or 1,
        import_mask=sum(1 << r.row for r in rows),
        row_generations=tuple(gens),
        block_ids=tuple(blocks),
        source_bytes=table.source_bytes,
        source_offsets=table.source_offsets,
        keys=table.keys,
        geometry=g,
    )
    transfer.validate()
    return transfer


def release_kv_device_exports(worker: Any) -> None:
    """Forget the worker's exports (HIP IPC handles need no close on the
    exporting side; importers close their mappings)."""
    worker._resident_epoch_device_kv_exports = None
