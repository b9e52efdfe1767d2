"""In-process engine: the resident epoch library called through ctypes in
the worker's own process.

Mirrors src/vllm_ascend_resident_epoch/ctypes_backend.py:30-254 (same
environment variables and outputs).  The library defaults to the one built
into this package when VLLM_ASCEND_RESIDENT_EPOCH_LIBRARY is unset.  Unlike
the reference's in-process engine this one also offers ``warm_up`` (the
sidecar's warm-up request, run directly).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Any

from . import _lib
from .backend import NativeEpochOutput, NativeWarmupOutput
from .contract import EpochCommitState, ResidentEpochExecutionError, ResidentEpochPlan
from .kv_transfer import DeviceKVTransfer, ResidentKVSnapshot, write_kv_snapshot
from .sidecar_backend import DEFAULT_EOS, WARMUP_GENERATION, WARMUP_TOKEN

MAX_EPOCH_STEPS = 8
ROWS = 4


def _env_path(name: str, *, directory: bool = False, default: Path | None = None) -> Path:
    raw = os.getenv(name)
    if not raw and default is None:
        raise RuntimeError(f"{name} is required by the resident epoch backend")
    path = Path(raw).resolve() if raw else default
    if not (path.is_dir() if directory else path.is_file()):
        raise RuntimeError(f"{name} must name an existing {'directory' if directory else 'file'}: {path}")
    return path


class CtypesDataFlowEngine:
    warmup_token = WARMUP_TOKEN
    warmup_eos = DEFAULT_EOS

    def __init__(self) -> None:
        library = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_LIBRARY", default=_lib.LIBRARY_PATH)
        air = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_AIR")
        graph_config = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_GRAPH_CONFIG")
        func_config = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_FUNC_CONFIG")
        tiling = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_TILING")
        weights = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_EXTERNAL_WEIGHTS", directory=True)
        if not str(weights).startswith("/dev/shm/"):
            raise RuntimeError("resident epoch external weights must be in /dev/shm")
        self.library = _lib.load(library)
        status = ctypes.c_int32(-1)
        self.handle = self.library.resident_epoch_create(
            str(air).encode(), str(graph_config).encode(), str(func_config).encode(), str(weights).encode(),
            str(tiling).encode(), ctypes.byref(status),
        )
        if not self.handle or status.value != 0:
            raise RuntimeError(f"failed to create the resident epoch engine, status={status.value}")

    def _call(self, count: int, steps: int, tokens, positions, lengths, eos, gens,
              transfer_path: Path | None, transfer_id: int, ipc: Any | None):
        """One resident_epoch_execute; returns (status, outputs)."""
        i64x4, i32x4 = ctypes.c_int64 * ROWS, ctypes.c_int32 * ROWS
        out = {
            "tokens": (ctypes.c_int64 * (ROWS * MAX_EPOCH_STEPS))(),
            "executed": i32x4(),
            "generations": i32x4(),
        }
        scalars = {k: ctypes.c_int32(v) for k, v in (("calls", 0), ("device", -1), ("feeds", 0), ("fetches", 0),
                                                       ("commit", -1), ("checksum", 0))}
        wide = {k: ctypes.c_int64(0) for k in ("wall", "cpu", "in_bytes", "out_bytes")}
        status = self.library.resident_epoch_execute(
            self.handle, count, steps, i64x4(*tokens), i64x4(*positions), i32x4(*lengths), i32x4(*eos),
            i32x4(*gens), out["tokens"], out["executed"], out["generations"],
            *(ctypes.byref(scalars[k]) for k in ("calls", "device", "feeds", "fetches", "commit", "checksum")),
            *(ctypes.byref(wide[k]) for k in ("wall", "cpu", "in_bytes", "out_bytes")),
            str(transfer_path).encode() if transfer_path is not None else None,
            transfer_id,
            ctypes.cast(ipc, ctypes.c_void_p) if ipc is not None else None,
        )
        try:
            commit = EpochCommitState(scalars["commit"].value)
        except ValueError as exc:
            raise ResidentEpochExecutionError(
                "resident_epoch_execute returned no valid commit state", commit_state=EpochCommitState.EXECUTING,
                status=status,
            ) from exc
        if status != 0:
            raise ResidentEpochExecutionError(
                f"resident_epoch_execute failed with status {status}", commit_state=commit, status=status
            )
        values = {k: v.value for k, v in {**scalars, **wide}.items()}
        values["commit"] = commit
        return out, values

    def warm_up(self) -> NativeWarmupOutput:
        _, v = self._call(1, 1, [self.warmup_token, 0, 0, 0], [0] * 4, [1, 0, 0, 0], [self.warmup_eos] * 4,
                          [WARMUP_GENERATION, 0, 0, 0], None, 0, None)
        return NativeWarmupOutput(
            status=v["device"], model_calls=v["calls"], feed_calls=v["feeds"], fetch_calls=v["fetches"],
            commit_state=v["commit"], wall_us=v["wall"], native_cpu_us=v["cpu"],
            declared_input_bytes=v["in_bytes"], declared_output_bytes=v["out_bytes"],
        )

    def execute(self, plan: ResidentEpochPlan) -> NativeEpochOutput:
        return self._execute(plan, transfer_path=None, transfer_id=0, ipc_metadata=None)

    def execute_with_import(self, plan: ResidentEpochPlan, snapshot: ResidentKVSnapshot) -> NativeEpochOutput:
        path = Path(f"/dev/shm/cruise-kv-transfer-{os.getpid()}-{snapshot.transfer_id}")
        write_kv_snapshot(path, snapshot)
        try:
            return self._execute(plan, transfer_path=path, transfer_id=snapshot.transfer_id, ipc_metadata=None)
        finally:
            path.unlink(missing_ok=True)

    def execute_with_device_transfer(self, plan: ResidentEpochPlan, transfer: DeviceKVTransfer) -> NativeEpochOutput:
        transfer.validate()
        record = ctypes.create_string_buffer(transfer.wire_bytes())
        return self._execute(plan, transfer_path=None, transfer_id=transfer.transfer_id, ipc_metadata=record)

    def _execute(self, plan: ResidentEpochPlan, *, transfer_path: Path | None, transfer_id: int,
                 ipc_metadata: Any | None) -> NativeEpochOutput:
        if plan.graph_batch_size != ROWS:
            raise ValueError("the ctypes backend owns only the static B=4 graph")
        fields = {"token_id": 0, "position": 0, "sequence_length": 0, "eos_token_id": DEFAULT_EOS}
        rows = {name: [fill] * ROWS for name, fill in fields.items()}
        for r in plan.requests:
            for name in fields:
                rows[name][r.row] = int(getattr(r, name))
        out, v = self._call(len(plan.requests), plan.max_steps, rows["token_id"], rows["position"],
                            rows["sequence_length"], rows["eos_token_id"], list(plan.row_generations),
                            transfer_path, transfer_id, ipc_metadata)
        tokens: dict[str, list[int]] = {}
        for r in plan.requests:
            n = out["executed"][r.row]
            if not 0 <= n <= plan.max_steps:
                raise ResidentEpochExecutionError("native backend returned an invalid executed count",
                                                  commit_state=v["commit"])
            tokens[r.req_id] = [int(out["tokens"][r.row * MAX_EPOCH_STEPS + s]) for s in range(n)]
        imported = transfer_path is not None or ipc_metadata is not None
        return NativeEpochOutput(
            status=v["device"], model_calls=v["calls"], token_ids=tokens, row_generations=tuple(out["generations"]),
            commit_state=v["commit"], feed_calls=v["feeds"], fetch_calls=v["fetches"], wall_us=v["wall"],
            native_cpu_us=v["cpu"], declared_input_bytes=v["in_bytes"], declared_output_bytes=v["out_bytes"],
            kv_imported=imported, kv_import_checksum=v["checksum"] & 0xFFFFFFFF,
        )

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
