"""Worker-side backend: runs one resident epoch through a native engine and
turns its output into a model-runner output with the epoch result attached.

Mirrors src/vllm_ascend_resident_epoch/backend.py:19-221.  A native engine
is anything with ``warm_up``, ``execute`` and optionally
``execute_with_import`` / ``execute_with_device_transfer``: the sidecar
client (sidecar_backend.py), the in-process ctypes engine
(ctypes_backend.py), or a test double.  Every failure is raised as a
ResidentEpochExecutionError carrying the commit state it reached.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field
from importlib import import_module
from typing import Protocol

from .contract import (
    CONTRACT_VERSION,
    EpochCommitState,
    ResidentEpochExecutionError,
    ResidentEpochPlan,
    ResidentEpochResult,
    attach_result,
)
from .kv_transfer import DeviceKVTransfer, ResidentKVSnapshot

try:  # the serving stack's output record when it is installed
    from vllm.v1.outputs import ModelRunnerOutput  # type: ignore
except ImportError:  # pragma: no cover - depends on the environment

    @dataclass
    class ModelRunnerOutput:  # type: ignore[no-redef]
        """The three fields of vLLM's ModelRunnerOutput an epoch fills."""

        req_ids: list[str]
        req_id_to_index: dict[str, int]
        sampled_token_ids: list[list[int]] = field(default_factory=list)


@dataclass(frozen=True)
class NativeEpochOutput:
    status: int
    model_calls: int
    token_ids: dict[str, list[int]]
    row_generations: tuple[int, ...]
    commit_state: EpochCommitState = EpochCommitState.COMMITTED
    feed_calls: int = 1
    fetch_calls: int = 1
    wall_us: int = 0
    native_cpu_us: int = 0
    declared_input_bytes: int = 0
    declared_output_bytes: int = 0
    socket_send_calls: int = 1
    socket_receive_calls: int = 1
    kv_imported: bool = False
    kv_import_checksum: int = 0
    kv_transfer_mode: str = "none"


@dataclass(frozen=True)
class NativeWarmupOutput:
    status: int
    model_calls: int
    feed_calls: int
    fetch_calls: int
    wall_us: int
    commit_state: EpochCommitState = EpochCommitState.COMMITTED
    native_cpu_us: int = 0
    declared_input_bytes: int = 0
    declared_output_bytes: int = 0
    socket_send_calls: int = 1
    socket_receive_calls: int = 1


class NativeEpochEngine(Protocol):
    def warm_up(self) -> NativeWarmupOutput: ...

    def execute(self, plan: ResidentEpochPlan) -> NativeEpochOutput: ...

    def execute_with_import(self, plan: ResidentEpochPlan, snapshot: ResidentKVSnapshot) -> NativeEpochOutput: ...

    def execute_with_device_transfer(self, plan: ResidentEpochPlan, transfer: DeviceKVTransfer) -> NativeEpochOutput: ...


class ResidentEpochBackend:
    def __init__(self, engine: NativeEpochEngine):
        self.engine = engine

    def warm_up(self) -> NativeWarmupOutput:
        out = self.engine.warm_up()
        if out.status != 0:
            raise RuntimeError(f"native resident warmup returned {out.status}")
        if (out.model_calls, out.feed_calls, out.fetch_calls) != (1, 1, 1) or out.commit_state != EpochCommitState.COMMITTED:
            raise RuntimeError("resident warmup must execute one complete decoder step")
        return out

    def close(self) -> None:
        close = getattr(self.engine, "close", None)
        if callable(close):
            close()

    def _run(self, plan, snapshot, device_transfer) -> NativeEpochOutput:
        """Dispatch to the engine; anything but an execution error becomes
        one in EXECUTING state (the device may have run)."""
        if device_transfer is not None:
            method, what, arg = "execute_with_device_transfer", "direct Device KV transfer", device_transfer
        elif snapshot is not None:
            method, what, arg = "execute_with_import", "KV import", snapshot
        else:
            method, what, arg = "execute", None, None
        try:
            fn = getattr(self.engine, method, None)
            if not callable(fn):
                raise ResidentEpochExecutionError(
                    f"resident backend does not support {what}", commit_state=EpochCommitState.PREPARED
                )
            return fn(plan) if arg is None else fn(plan, arg)
        except ResidentEpochExecutionError:
            raise
        except Exception as exc:
            raise ResidentEpochExecutionError(
                "native resident epoch failed without commit-state proof", commit_state=EpochCommitState.EXECUTING
            ) from exc

    def execute(
        self,
        plan: ResidentEpochPlan,
        snapshot: ResidentKVSnapshot | None = None,
        device_transfer: DeviceKVTransfer | None = None,
    ) -> ModelRunnerOutput:
        if snapshot is not None and device_transfer is not None:
            raise ValueError("resident epoch cannot use two KV transfer modes")
        try:
            plan.validate()
        except Exception as exc:
            raise ResidentEpochExecutionError(
                f"resident epoch plan validation failed: {exc}", commit_state=EpochCommitState.PREPARED
            ) from exc
        out = self._run(plan, snapshot, device_transfer)
        if out.status != 0:
            raise ResidentEpochExecutionError(
                f"native resident epoch returned status {out.status}", commit_state=out.commit_state, status=out.status
            )
        if out.commit_state != EpochCommitState.COMMITTED:
            raise ResidentEpochExecutionError(
                "successful native resident epoch was not committed", commit_state=out.commit_state
            )
        committed = EpochCommitState.COMMITTED
        if snapshot is not None and out.kv_import_checksum != snapshot.checksum:
            raise ResidentEpochExecutionError(
                "resident KV import checksum disagrees with the Host snapshot", commit_state=committed
            )
        if device_transfer is not None and out.kv_import_checksum == 0:
            raise ResidentEpochExecutionError(
                "direct Device KV transfer did not return an import checksum", commit_state=committed
            )
        if set(out.token_ids) != set(plan.req_ids):
            raise ResidentEpochExecutionError("native resident epoch returned the wrong request set", commit_state=committed)

        req_ids = list(plan.req_ids)
        sampled = {rid: list(out.token_ids[rid]) for rid in req_ids}
        mode = "device_ipc" if device_transfer is not None else ("host_snapshot" if snapshot is not None else "none")
        result = ResidentEpochResult(
            version=CONTRACT_VERSION,
            route="device",
            status=0,
            model_calls=out.model_calls,
            computed_steps={rid: len(sampled[rid]) for rid in req_ids},
            row_generations=out.row_generations,
            commit_state=out.commit_state,
            feed_calls=out.feed_calls,
            fetch_calls=out.fetch_calls,
            wall_us=out.wall_us,
            native_cpu_us=out.native_cpu_us,
            declared_input_bytes=out.declared_input_bytes,
            declared_output_bytes=out.declared_output_bytes,
            socket_send_calls=out.socket_send_calls,
            socket_receive_calls=out.socket_receive_calls,
            kv_imported=out.kv_imported,
            kv_import_checksum=out.kv_import_checksum,
            kv_snapshot_checksum=snapshot.checksum if snapshot is not None else 0,
            kv_transfer_mode=mode,
        )
        try:
            result.validate_against(plan, sampled)
        except Exception as exc:
            raise ResidentEpochExecutionError(
                f"committed resident epoch result is invalid: {exc}", commit_state=committed
            ) from exc
        output = ModelRunnerOutput(
            req_ids=req_ids,
            req_id_to_index={rid: i for i, rid in enumerate(req_ids)},
            sampled_token_ids=[sampled[rid] for rid in req_ids],
        )
        attach_result(output, result)
        return output


def load_backend_from_env() -> ResidentEpochBackend:
    """Build the backend from VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY =
    "module:factory" (backend.py:211-221), e.g.
    "cruise_amd.sidecar_backend:create_sidecar_engine"."""
    target = os.getenv("VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY")
    if not target or ":" not in target:
        raise RuntimeError(
            "VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY must name a module:factory for the native epoch backend"
        )
    module, factory = target.split(":", 1)
    return ResidentEpochBackend(getattr(import_module(module), factory)())
