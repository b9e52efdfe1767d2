"""In-process engine: the resident epoch library called through ctypes in
the worker's own process.

Same environment variables and outputs as
src/vllm_ascend_resident_epoch/ctypes_backend.py:30-254
(VLLM_ASCEND_RESIDENT_EPOCH_{LIBRARY, AIR, GRAPH_CONFIG, FUNC_CONFIG, TILING,
EXTERNAL_WEIGHTS}).  The library defaults to the one built into this package.
The plan travels as the shared per-row feed (epoch_io.py) and the outputs of
one resident_epoch_execute call come back as the shared fetch record, so this
engine and the sidecar client decode results identically.  Unlike the
reference's in-process engine this one also offers ``warm_up``.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Any

from . import _lib
from .backend import NativeEpochOutput, NativeWarmupOutput
from .contract import ResidentEpochPlan
from .epoch_io import DEFAULT_EOS, MAX_EPOCH_STEPS, ROWS, WARMUP_TOKEN, EpochFeed, EpochFetch, check_transfer
from .kv_transfer import DeviceKVTransfer, ResidentKVSnapshot, write_kv_snapshot

ENV = "VLLM_ASCEND_RESIDENT_EPOCH_"


def _existing(name: str, *, directory: bool = False, default: Path | None = None) -> Path:
    raw = os.getenv(ENV + name)
    if not raw and default is None:
        raise RuntimeError(f"{ENV}{name} must be set for the in-process resident epoch engine")
    path = Path(raw).resolve() if raw else default
    if not (path.is_dir() if directory else path.is_file()):
        raise RuntimeError(f"{ENV}{name}: {path} is not an existing {'directory' if directory else 'file'}")
    return path


class _Outputs:
    """The output arguments of resident_epoch_execute, in signature order."""

    ORDER = ("history", "executed", "generations", "model_calls", "device_status", "feed_calls", "fetch_calls",
             "commit_state", "checksum", "wall_us", "native_cpu_us", "declared_input_bytes",
             "declared_output_bytes")

    def __init__(self) -> None:
        self.history = (ctypes.c_int64 * (ROWS * MAX_EPOCH_STEPS))()
        self.executed = (ctypes.c_int32 * ROWS)()
        self.generations = (ctypes.c_int32 * ROWS)()
        for name in self.ORDER[3:9]:
            setattr(self, name, ctypes.c_int32(-1 if name in ("commit_state", "device_status") else 0))
        for name in self.ORDER[9:]:
            setattr(self, name, ctypes.c_int64(0))

    def arguments(self) -> list:
        return [getattr(self, name) if name in self.ORDER[:3] else ctypes.byref(getattr(self, name))
                for name in self.ORDER]

    def value(self, name: str) -> int:
        return getattr(self, name).value


class CtypesDataFlowEngine:
    warmup_token = WARMUP_TOKEN
    warmup_eos = DEFAULT_EOS

    def __init__(self) -> None:
        library = _existing("LIBRARY", default=_lib.LIBRARY_PATH)
        args = (_existing("AIR"), _existing("GRAPH_CONFIG"), _existing("FUNC_CONFIG"),
                _existing("EXTERNAL_WEIGHTS", directory=True), _existing("TILING"))
        if not str(args[3]).startswith("/dev/shm/"):
            raise RuntimeError(f"the external weight directory must be under /dev/shm, got {args[3]}")
        self.library = _lib.load_bridge(library)
        status = ctypes.c_int32(-1)
        self.handle = self.library.resident_epoch_create(*(str(a).encode() for a in args), ctypes.byref(status))
        if not self.handle or status.value != 0:
            raise RuntimeError(f"resident_epoch_create failed with status {status.value}")

    def _call(self, feed: EpochFeed, transfer_path: Path | None = None, transfer_id: int = 0,
              ipc: Any | None = None) -> EpochFetch:
        out = _Outputs()
        rows64, rows32 = ctypes.c_int64 * ROWS, ctypes.c_int32 * ROWS
        status = self.library.resident_epoch_execute(
            self.handle, feed.request_count, feed.max_steps, rows64(*feed.tokens), rows64(*feed.positions),
            rows32(*feed.lengths), rows32(*feed.eos), rows32(*feed.generations), *out.arguments(),
            str(transfer_path).encode() if transfer_path is not None else None, transfer_id,
            ctypes.cast(ipc, ctypes.c_void_p) if ipc is not None else None,
        )
        return EpochFetch(
            transport_status=status, device_status=out.value("device_status"), model_calls=out.value("model_calls"),
            feed_calls=out.value("feed_calls"), fetch_calls=out.value("fetch_calls"),
            commit_code=out.value("commit_state"), checksum=out.value("checksum"), wall_us=out.value("wall_us"),
            native_cpu_us=out.value("native_cpu_us"), declared_input_bytes=out.value("declared_input_bytes"),
            declared_output_bytes=out.value("declared_output_bytes"),
            executed=tuple(out.executed), generations=tuple(out.generations), history=tuple(out.history),
            source="resident_epoch_execute",
        )

    def warm_up(self) -> NativeWarmupOutput:
        return self._call(EpochFeed.warm_up(self.warmup_token, self.warmup_eos)).warmup_output()

    def execute(self, plan: ResidentEpochPlan) -> NativeEpochOutput:
        return self._call(EpochFeed.from_plan(plan)).native_output(plan)

    def execute_with_import(self, plan: ResidentEpochPlan, snapshot: ResidentKVSnapshot) -> NativeEpochOutput:
        snapshot.validate()
        check_transfer(plan, snapshot.import_mask, snapshot.row_generations, "KV snapshot")
        path = Path(f"/dev/shm/cruise-kv-transfer-{os.getpid()}-{snapshot.transfer_id}")
        write_kv_snapshot(path, snapshot)
        try:
            fetch = self._call(EpochFeed.from_plan(plan), path, snapshot.transfer_id)
        finally:
            path.unlink(missing_ok=True)
        return fetch.native_output(plan, "host_snapshot")

    def execute_with_device_transfer(self, plan: ResidentEpochPlan, transfer: DeviceKVTransfer) -> NativeEpochOutput:
        transfer.validate()
        check_transfer(plan, transfer.import_mask, transfer.row_generations, "device KV transfer")
        record = ctypes.create_string_buffer(transfer.wire_bytes())
        return self._call(EpochFeed.from_plan(plan), None, transfer.transfer_id, record).native_output(plan,
                                                                                                     "device_ipc")

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.library.resident_epoch_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def create_ctypes_engine() -> CtypesDataFlowEngine:
    return CtypesDataFlowEngine()
