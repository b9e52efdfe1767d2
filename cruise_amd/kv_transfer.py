"""Handing a prefilled row's KV to the resident epoch.

A row that was prefilled outside the device program (stock prefill into a
paged cache) becomes device-owned by importing its first KV block of every
layer: positions 0..block_size-1, the only block a prompt that fits the
epoch's window occupies.  Two transports exist:

* **host snapshot** -- the selected blocks travel through a file under
  /dev/shm that the engine reads into the epoch's one feed copy;
* **device IPC** -- only a 4,088-byte record crosses the process boundary:
  one HIP IPC handle per K and V cache of every layer, each cache's offset in
  its allocation, and the scheduler block of every imported row.  The engine
  maps the handles once and gathers the blocks on the device.

What must match the engine and the reference's callers byte for byte, and is
kept for that reason only (src/vllm_ascend_resident_epoch/kv_transfer.py:
14-34, 159-174):

* the 80-byte snapshot header ``<QIIQQI4i7I`` (magic "CRUISEKV", version 1)
  followed by the payload ``[K | V][layer][row][block]``;
* the IPC record: header ``<QIIQ4i4i56Q`` (magic "CRUISEIP", version 2) and
  56 key slots of 64 bytes;
* the payload checksum: Adler-32 over the selected rows' blocks, K before V,
  layer-major, rows ascending.  The device recomputes it over the bytes it
  imported and the host compares.

A HIP IPC handle (``hipIpcMemHandle_t``) is a 64-byte binary record, so a
key slot holds those 64 bytes where an Ascend key was an ASCII name.

The rest is this module's own:

* the checksum is one ``zlib.adler32`` over a fancy-indexed numpy view
  ``payload[:, :, rows]``, whose C order is exactly the order above;
* both transfers validate through one rule table each (``TransferError``
  names the broken rule), sharing the row-selection rules;
* a snapshot is gathered on the caches' device with ``index_select`` and
  reaches the host as one copy per cache (K, V) for all layers;
* the snapshot file is written through ``mkstemp`` in the target directory,
  fsynced and renamed into place, so a reader never sees a partial file and
  concurrent writers never collide;
* IPC exports live in a small registry keyed by the caches' addresses and
  their allocations, so a moved or reallocated cache is exported afresh.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import secrets
import struct
import tempfile
import zlib
from collections import OrderedDict
from dataclasses import dataclass, field
from functools import lru_cache
from pathlib import Path
from typing import Any, Callable, Iterable

import numpy as np

TRANSFER_MAGIC = 0x4352554953454B56  # "CRUISEKV"
TRANSFER_VERSION = 1
TRANSFER_HEADER_BYTES = 80
IPC_METADATA_MAGIC = 0x4352554953454950  # "CRUISEIP"
IPC_METADATA_VERSION = 2
IPC_KEY_BYTES = 64  # sizeof(hipIpcMemHandle_t)


@dataclass(frozen=True)
class KVGeometry:
    """Shape of the imported blocks; Qwen2.5-7B at B=4 by default."""

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
        """Bytes of the K (or V) half of a payload."""
        return self.layers * self.batch * self.block_bytes

    @property
    def payload_bytes(self) -> int:
        return 2 * self.cache_bytes

    @property
    def key_count(self) -> int:
        """Caches a device transfer names: K and V of every layer."""
        return 2 * self.layers


QWEN7B_B4 = KVGeometry()

# The reference geometry's sizes, as its callers import them.
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

HEADER = struct.Struct("<QIIQQI4i7I")
IPC_METADATA_HEADER = struct.Struct(f"<QIIQ4i4i{IPC_KEY_COUNT}Q")
IPC_METADATA_BYTES = IPC_METADATA_HEADER.size + IPC_KEY_COUNT * IPC_KEY_BYTES
assert HEADER.size == TRANSFER_HEADER_BYTES and IPC_METADATA_BYTES == 4088


class TransferError(ValueError):
    """A transfer record broke one of its rules (``rule`` names it)."""

    def __init__(self, rule: str, detail: str):
        super().__init__(f"{detail} [{rule}]")
        self.rule = rule


Rule = tuple[str, Callable[[Any], bool], str]


def _enforce(rules: Iterable[Rule], record: Any) -> None:
    for name, holds, detail in rules:
        if not holds(record):
            raise TransferError(name, detail)


# ---------------------------------------------------------------------------
# Payload view and checksum
# ---------------------------------------------------------------------------
def selected_rows(mask: int, batch: int) -> list[int]:
    return [row for row in range(batch) if mask >> row & 1]


def payload_blocks(payload: bytes, geometry: KVGeometry) -> np.ndarray:
    """The payload as uint8 [2 (K, V), layers, batch, block_bytes]."""
    g = geometry
    if len(payload) != g.payload_bytes:
        raise TransferError("payload-size", f"a payload of this geometry has {g.payload_bytes} bytes, not {len(payload)}")
    return np.frombuffer(payload, dtype=np.uint8).reshape(2, g.layers, g.batch, g.block_bytes)


def kv_payload_checksum(payload: bytes, import_mask: int, geometry: KVGeometry = QWEN7B_B4) -> int:
    """Adler-32 of the selected rows' blocks, K before V, layer-major, rows
    ascending: the C order of ``blocks[:, :, rows]``."""
    rows = selected_rows(import_mask, geometry.batch)
    picked = np.ascontiguousarray(payload_blocks(payload, geometry)[:, :, rows])
    return zlib.adler32(memoryview(picked).cast("B")) & 0xFFFFFFFF


# ---------------------------------------------------------------------------
# Row selection, shared by both transfers
# ---------------------------------------------------------------------------
def _selection_rules(batch_of: Callable[[Any], int]) -> tuple[Rule, ...]:
    return (
        ("transfer-id", lambda t: t.transfer_id > 0, "a transfer id is a positive integer"),
        ("generation-count", lambda t: len(t.row_generations) == batch_of(t),
         "the generation vector has one entry per graph row"),
        ("mask-range", lambda t: 0 < t.import_mask < 1 << batch_of(t),
         "the import mask selects one or more of the graph's rows and nothing else"),
        ("generation-sign", lambda t: min(t.row_generations) >= 0, "generations are never negative"),
    )


# ---------------------------------------------------------------------------
# Host snapshot
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class ResidentKVSnapshot:
    """The selected rows' blocks copied to the host, with their checksum
    (unselected rows' blocks are zero)."""

    transfer_id: int
    import_mask: int
    row_generations: tuple[int, ...]
    payload: bytes
    checksum: int
    geometry: KVGeometry = field(default=QWEN7B_B4)

    RULES = _selection_rules(lambda s: s.geometry.batch) + (
        ("generation-selects-row",
         lambda s: all((s.import_mask >> r & 1) == (gen > 0) for r, gen in enumerate(s.row_generations)),
         "exactly the rows with a generation are selected"),
        ("payload-size", lambda s: len(s.payload) == s.geometry.payload_bytes,
         "the payload holds every row's block of every layer, K then V"),
        ("checksum", lambda s: s.checksum == kv_payload_checksum(s.payload, s.import_mask, s.geometry),
         "the checksum is not the payload's"),
    )

    def validate(self) -> None:
        _enforce(self.RULES, self)

    def header(self) -> bytes:
        g = self.geometry
        return HEADER.pack(
            TRANSFER_MAGIC, TRANSFER_VERSION, TRANSFER_HEADER_BYTES, self.transfer_id, len(self.payload),
            self.import_mask, *self.row_generations,
            g.layers, g.batch, g.block_size, g.kv_heads, g.head_size, g.element_bytes, self.checksum,
        )

    @classmethod
    def parse(cls, raw: bytes) -> "ResidentKVSnapshot":
        if len(raw) < TRANSFER_HEADER_BYTES:
            raise TransferError("file-size", "the file ends inside its header")
        magic, version, header_bytes, transfer_id, payload_bytes, mask, *rest = HEADER.unpack_from(raw)
        gens, dims, checksum = tuple(rest[:4]), rest[4:10], rest[10]
        if (magic, version, header_bytes) != (TRANSFER_MAGIC, TRANSFER_VERSION, TRANSFER_HEADER_BYTES):
            raise TransferError("magic", "not a version-1 KV snapshot file")
        if len(raw) != header_bytes + payload_bytes:
            raise TransferError("file-size", "the file size disagrees with its header")
        snapshot = cls(transfer_id, mask, gens, bytes(raw[header_bytes:]), checksum, KVGeometry(*dims))
        snapshot.validate()
        return snapshot


def _under_dev_shm(path: Path) -> bool:
    return path.parts[:3] == ("/", "dev", "shm") and len(path.parts) > 3


def write_kv_snapshot(path: str | Path, snapshot: ResidentKVSnapshot) -> None:
    """Publish a snapshot at ``path`` (under /dev/shm, where the engine reads
    transfer files): written to a fresh temporary file in the same directory,
    fsynced, then renamed over ``path``."""
    snapshot.validate()
    target = Path(path).resolve()
    if not _under_dev_shm(target):
        raise TransferError("location", f"the engine reads transfer files under /dev/shm only, not {target}")
    target.parent.mkdir(parents=True, exist_ok=True)
    fd, staging = tempfile.mkstemp(dir=target.parent, prefix=f".{target.name}.", suffix=".partial")
    try:
        with os.fdopen(fd, "wb") as out:
            out.write(snapshot.header())
            out.write(snapshot.payload)
            out.flush()
            os.fsync(out.fileno())
        os.replace(staging, target)
    except BaseException:
        with contextlib.suppress(FileNotFoundError):
            os.unlink(staging)
        raise


def read_kv_snapshot(path: str | Path) -> ResidentKVSnapshot:
    return ResidentKVSnapshot.parse(Path(path).read_bytes())


# ---------------------------------------------------------------------------
# Device IPC record
# ---------------------------------------------------------------------------
def _blocks_inside_sources(t: "DeviceKVTransfer") -> bool:
    block = t.geometry.block_bytes
    ends = [(t.block_ids[r] + 1) * block for r in selected_rows(t.import_mask, t.geometry.batch)]
    return all(0 <= off and off + end <= t.source_bytes for off in t.source_offsets for end in ends)


def _rows_consistent(t: "DeviceKVTransfer") -> bool:
    for row, (gen, block) in enumerate(zip(t.row_generations, t.block_ids)):
        if t.import_mask >> row & 1:
            if gen <= 0 or block < 0:
                return False
        elif gen != 0 or block != 0:
            return False
    return True


@dataclass(frozen=True)
class DeviceKVTransfer:
    """A device-to-device import, as metadata only.

    ``keys[2 l]`` / ``keys[2 l + 1]``: the IPC handle of the allocation that
    holds layer l's K / V cache, at byte ``source_offsets[...]`` of it;
    ``source_bytes``: the size every such allocation has; ``block_ids``: the
    stock cache block of each selected row (0 for the others)."""

    transfer_id: int
    import_mask: int
    row_generations: tuple[int, ...]
    block_ids: tuple[int, ...]
    source_bytes: int
    source_offsets: tuple[int, ...]
    keys: tuple[bytes, ...]
    geometry: KVGeometry = field(default=QWEN7B_B4)

    RULES = _selection_rules(lambda t: t.geometry.batch) + (
        ("record-capacity", lambda t: t.geometry.key_count <= IPC_KEY_COUNT,
         f"the record has key slots for {IPC_KEY_COUNT // 2} layers"),
        ("block-count", lambda t: len(t.block_ids) == t.geometry.batch, "the block vector has one entry per graph row"),
        ("source-size", lambda t: t.source_bytes > 0, "the exported allocations have a size"),
        ("offset-count", lambda t: len(t.source_offsets) == t.geometry.key_count,
         "one source offset per K and V cache of every layer"),
        ("key-count", lambda t: len(t.keys) == t.geometry.key_count, "one key per K and V cache of every layer"),
        ("row-fields", _rows_consistent,
         "a selected row carries a generation and a block; an unselected row carries zeros"),
        ("block-range", _blocks_inside_sources, "a selected block lies past the end of an exported allocation"),
        ("key-format", lambda t: all(isinstance(k, (bytes, bytearray)) and len(k) == IPC_KEY_BYTES and any(k)
                                     for k in t.keys),
         f"a key is a nonzero {IPC_KEY_BYTES}-byte IPC handle"),
    )

    def validate(self) -> None:
        _enforce(self.RULES, self)

    def wire_bytes(self) -> bytes:
        """The 4,088-byte record the engine reads (``ResidentEpochIpcMetadata``);
        the slots of layers a smaller geometry lacks stay zero."""
        self.validate()
        unused = IPC_KEY_COUNT - len(self.keys)
        record = bytearray(IPC_METADATA_BYTES)
        IPC_METADATA_HEADER.pack_into(
            record, 0, IPC_METADATA_MAGIC, IPC_METADATA_VERSION, self.import_mask, self.source_bytes,
            *self.row_generations, *self.block_ids, *self.source_offsets, *([0] * unused),
        )
        for slot, key in enumerate(self.keys):
            start = IPC_METADATA_HEADER.size + slot * IPC_KEY_BYTES
            record[start : start + IPC_KEY_BYTES] = key
        return bytes(record)


# ---------------------------------------------------------------------------
# Reading a worker's stock caches
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class _Import:
    row: int
    block: int
    generation: int


def _imports_of(plan: Any, what: str) -> list[_Import]:
    picked = []
    for request in plan.requests:
        if not request.kv_import_required:
            continue
        if len(request.scheduler_block_ids) != 1:
            raise TransferError("one-block", f"{what}: an imported row occupies exactly one stock block")
        picked.append(_Import(request.row, int(request.scheduler_block_ids[0]), int(request.generation)))
    if not picked:
        raise TransferError("no-imports", f"{what}: the plan imports no row")
    return sorted(picked, key=lambda i: i.row)


def _cache_pairs(worker: Any) -> list[tuple[Any, Any]]:
    """(K, V) per layer from ``worker.model_runner.kv_caches``."""
    layers = getattr(getattr(worker, "model_runner", None), "kv_caches", None)
    if not isinstance(layers, list) or not layers:
        raise RuntimeError("the worker holds no per-layer stock KV caches")
    pairs = []
    for layer in layers:
        if not isinstance(layer, (tuple, list)) or len(layer) < 2:
            raise RuntimeError("a stock KV cache layer is not a (K, V) pair")
        pairs.append((layer[0], layer[1]))
    return pairs


def _geometry(pairs: list[tuple[Any, Any]], batch: int) -> KVGeometry:
    key = pairs[0][0]
    if key.dim() != 4:
        raise RuntimeError("stock KV caches are laid out [blocks, block_size, kv_heads, head]")
    _, block_size, kv_heads, head = (int(s) for s in key.shape)
    return KVGeometry(len(pairs), batch, block_size, kv_heads, head, int(key.element_size()))


def _fresh_transfer_id() -> int:
    return secrets.randbits(63) or 1


def _import_fields(imports: list[_Import], batch: int) -> tuple[int, tuple[int, ...], tuple[int, ...]]:
    gens, blocks = [0] * batch, [0] * batch
    for i in imports:
        gens[i.row], blocks[i.row] = i.generation, i.block
    return sum(1 << i.row for i in imports), tuple(gens), tuple(blocks)


def capture_kv_snapshot(worker: Any, plan: Any, batch: int | None = None) -> ResidentKVSnapshot:
    """Copy each imported row's stock block of every layer into a snapshot.

    The blocks are gathered where the caches live (one ``index_select`` per
    layer and cache) and copied to the host once per cache (K, then V)."""
    import torch

    imports = _imports_of(plan, "KV snapshot")
    pairs = _cache_pairs(worker)
    g = _geometry(pairs, batch or plan.graph_batch_size)
    if plan.logical_capacity > g.block_size:
        raise TransferError("window", "a snapshot carries one block per row: the epoch's window must fit in it")
    dtype = pairs[0][0].dtype
    blocks = torch.tensor([i.block for i in imports], dtype=torch.int64)
    rows = [i.row for i in imports]
    out = np.zeros((2, g.layers, g.batch, g.block_bytes), dtype=np.uint8)
    for half in range(2):
        caches = [pair[half] for pair in pairs]
        if any(c.dtype != dtype or tuple(c.shape[1:]) != tuple(caches[0].shape[1:]) for c in caches):
            raise TransferError("cache-format", "every stock cache shares one dtype and block shape")
        if any(not 0 <= i.block < c.shape[0] for c in caches for i in imports):
            raise TransferError("block-range", "an imported block lies outside its stock cache")
        index = blocks.to(caches[0].device)
        gathered = torch.stack([c.detach().index_select(0, index) for c in caches])  # [layers, rows, block...]
        host = gathered.contiguous().cpu().view(torch.uint8).numpy()
        out[half][:, rows] = host.reshape(g.layers, len(rows), g.block_bytes)
    payload = out.tobytes()
    mask, gens, _ = _import_fields(imports, g.batch)
    snapshot = ResidentKVSnapshot(_fresh_transfer_id(), mask, gens, payload, kv_payload_checksum(payload, mask, g), g)
    snapshot.validate()
    return snapshot


# ---------------------------------------------------------------------------
# Device IPC exports
# ---------------------------------------------------------------------------
@lru_cache(maxsize=1)
def _hip() -> ctypes.CDLL:
    lib = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
    lib.hipMemGetAddressRange.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t), ctypes.c_void_p]
    lib.hipMemGetAddressRange.restype = ctypes.c_int
    lib.hipIpcGetMemHandle.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.hipIpcGetMemHandle.restype = ctypes.c_int
    return lib


def _allocation_of(address: int) -> tuple[int, int]:
    """(base, size) of the device allocation that contains ``address``."""
    base, size = ctypes.c_void_p(), ctypes.c_size_t()
    rc = _hip().hipMemGetAddressRange(ctypes.byref(base), ctypes.byref(size), ctypes.c_void_p(address))
    if rc != 0 or not base.value or not size.value:
        raise RuntimeError(f"hipMemGetAddressRange found no allocation for a stock KV cache (error {rc})")
    return int(base.value), int(size.value)


def _ipc_handle(base: int) -> bytes:
    handle = ctypes.create_string_buffer(IPC_KEY_BYTES)
    rc = _hip().hipIpcGetMemHandle(handle, ctypes.c_void_p(base))
    if rc != 0:
        raise RuntimeError(f"hipIpcGetMemHandle refused a stock KV allocation (error {rc})")
    return handle.raw


@dataclass(frozen=True)
class _Exports:
    source_bytes: int
    source_offsets: tuple[int, ...]
    keys: tuple[bytes, ...]


class _ExportRegistry:
    """IPC exports of stock KV allocations, one handle per allocation.

    Entries are keyed by every cache's (address, allocation base, allocation
    size), so caches that move or whose memory is reallocated get new
    handles; a handle stays valid while its allocation lives.  The registry
    keeps the most recent few cache sets."""

    def __init__(self, limit: int = 4):
        self.limit = limit
        self.entries: OrderedDict[tuple, _Exports] = OrderedDict()

    @staticmethod
    def _placement(tensors: list[Any]) -> tuple[tuple[int, int, int], ...]:
        placement = []
        for t in tensors:
            if not getattr(t, "is_cuda", False) or not t.is_contiguous():
                raise RuntimeError("IPC export needs contiguous device tensors for the stock KV caches")
            address = int(t.data_ptr())
            base, size = _allocation_of(address)
            if address + t.numel() * t.element_size() > base + size:
                raise RuntimeError("a stock KV cache runs past the end of its allocation")
            placement.append((address, base, size))
        return tuple(placement)

    def exports(self, tensors: list[Any]) -> _Exports:
        placement = self._placement(tensors)
        found = self.entries.get(placement)
        if found is not None:
            self.entries.move_to_end(placement)
            return found
        sizes = {size for _, _, size in placement}
        if len(sizes) != 1:
            raise RuntimeError("the stock KV allocations differ in size; the record carries one size")
        handles = {base: _ipc_handle(base) for base in dict.fromkeys(base for _, base, _ in placement)}
        made = _Exports(sizes.pop(), tuple(a - b for a, b, _ in placement), tuple(handles[b] for _, b, _ in placement))
        self.entries[placement] = made
        while len(self.entries) > self.limit:
            self.entries.popitem(last=False)
        return made

    def forget(self, tensors: list[Any]) -> None:
        addresses = tuple(int(t.data_ptr()) for t in tensors)
        for placement in [p for p in self.entries if tuple(a for a, _, _ in p) == addresses]:
            del self.entries[placement]


_REGISTRY = _ExportRegistry()


def _flat_caches(pairs: list[tuple[Any, Any]]) -> list[Any]:
    return [t for pair in pairs for t in pair]


def capture_kv_device_transfer(worker: Any, plan: Any, batch: int | None = None) -> DeviceKVTransfer:
    """The IPC record that imports the plan's rows; no KV byte leaves the
    device."""
    imports = _imports_of(plan, "device KV transfer")
    pairs = _cache_pairs(worker)
    g = _geometry(pairs, batch or plan.graph_batch_size)
    exports = _REGISTRY.exports(_flat_caches(pairs))
    mask, gens, blocks = _import_fields(imports, g.batch)
    transfer = DeviceKVTransfer(_fresh_transfer_id(), mask, gens, blocks, exports.source_bytes,
                                exports.source_offsets, exports.keys, g)
    transfer.validate()
    return transfer


def release_kv_device_exports(worker: Any) -> None:
    """Drop the exports of the worker's current caches (the exporting side
    closes nothing; importers unmap their own mappings)."""
    with contextlib.suppress(RuntimeError):
        _REGISTRY.forget(_flat_caches(_cache_pairs(worker)))
