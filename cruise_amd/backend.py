"""Worker side of a resident epoch: run a plan through a native engine and
return the model-runner output with the epoch result attached.

Interface kept from src/vllm_ascend_resident_epoch/backend.py: the engine
protocol (``warm_up``, ``execute`` and the optional ``execute_with_import``
/ ``execute_with_device_transfer``, 54-67), the records engines return
(``NativeEpochOutput``, ``NativeWarmupOutput``, 19-51), ``ResidentEpochBackend``
with ``warm_up`` / ``execute`` / ``close``, and ``load_backend_from_env``
reading VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY = "module:factory"
(211-221).  The commit-state semantics are the contract's (backend.py:90-208):
a failure before the engine is called is PREPARED, an engine call that fails
without saying how far it got is EXECUTING, and anything wrong with a
successful engine answer is COMMITTED.

Here those semantics are the structure of ``execute``: it walks through
three stages, and the stage guard ``_stage`` turns any exception raised in a
stage into a ResidentEpochExecutionError at that stage's commit state
(errors that already carry a commit state pass through unchanged).
"""
from __future__ import annotations

import os
from contextlib import contextmanager
from dataclasses import dataclass, field
from importlib import import_module
from typing import Callable, Iterator, Protocol

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


@contextmanager
def _stage(state: EpochCommitState, what: str) -> Iterator[None]:
    """Run a stage of an epoch: an exception raised in it becomes an
    execution error at ``state``, unless it already is one."""
    try:
        yield
    except ResidentEpochExecutionError:
        raise
    except Exception as exc:
        raise ResidentEpochExecutionError(f"{what}: {exc}", commit_state=state) from exc


@dataclass(frozen=True)
class _Transfer:
    """How an epoch's KV arrives: not at all, as a host snapshot file, or
    over device IPC; names the engine method that performs it."""

    mode: str
    method: str
    argument: object = None

    @classmethod
    def choose(cls, snapshot: ResidentKVSnapshot | None, device: DeviceKVTransfer | None) -> "_Transfer":
        if snapshot is not None and device is not None:
            raise ValueError("an epoch takes its KV from one source: a host snapshot or a device IPC transfer")
        if device is not None:
            return cls("device_ipc", "execute_with_device_transfer", device)
        if snapshot is not None:
            return cls("host_snapshot", "execute_with_import", snapshot)
        return cls("none", "execute")

    def bind(self, engine: object) -> Callable[[ResidentEpochPlan], NativeEpochOutput]:
        method = getattr(engine, self.method, None)
        if not callable(method):
            raise ResidentEpochExecutionError(f"the engine has no {self.method} for a {self.mode} KV transfer",
                                              commit_state=EpochCommitState.PREPARED)
        if self.argument is None:
            return method
        return lambda plan: method(plan, self.argument)

    def check_proof(self, out: NativeEpochOutput) -> None:
        """The checksum an import returns must prove the transfer: equal to
        the snapshot's for a host snapshot, non-zero over device IPC."""
        if self.mode == "host_snapshot" and out.kv_import_checksum != self.argument.checksum:
            raise ValueError(f"imported KV checksum {out.kv_import_checksum:#010x} disagrees with the host "
                             f"snapshot's {self.argument.checksum:#010x}")
        if self.mode == "device_ipc" and out.kv_import_checksum == 0:
            raise ValueError("a device IPC import returned no checksum")

    @property
    def snapshot_checksum(self) -> int:
        return self.argument.checksum if self.mode == "host_snapshot" else 0


def _device_result(plan: ResidentEpochPlan, out: NativeEpochOutput, transfer: _Transfer) -> ResidentEpochResult:
    return ResidentEpochResult(
        version=CONTRACT_VERSION, route="device", status=0, model_calls=out.model_calls,
        computed_steps={rid: len(out.token_ids[rid]) for rid in plan.req_ids},
        row_generations=tuple(out.row_generations), commit_state=out.commit_state,
        feed_calls=out.feed_calls, fetch_calls=out.fetch_calls, wall_us=out.wall_us,
        native_cpu_us=out.native_cpu_us, declared_input_bytes=out.declared_input_bytes,
        declared_output_bytes=out.declared_output_bytes, socket_send_calls=out.socket_send_calls,
        socket_receive_calls=out.socket_receive_calls, kv_imported=out.kv_imported,
        kv_import_checksum=out.kv_import_checksum, kv_snapshot_checksum=transfer.snapshot_checksum,
        kv_transfer_mode=transfer.mode,
    )


class ResidentEpochBackend:
    def __init__(self, engine: NativeEpochEngine):
        self.engine = engine

    def warm_up(self) -> NativeWarmupOutput:
        """The engine's warm-up must be one complete, committed decoder step
        with one feed and one fetch."""
        out = self.engine.warm_up()
        if out.status != 0:
            raise RuntimeError(f"the engine's warm-up failed with device status {out.status}")
        shape = (out.model_calls, out.feed_calls, out.fetch_calls, out.commit_state)
        if shape != (1, 1, 1, EpochCommitState.COMMITTED):
            raise RuntimeError(f"a warm-up is one complete decoder step (calls, feeds, fetches, state = 1, 1, 1, "
                               f"COMMITTED), the engine did {shape}")
        return out

    def close(self) -> None:
        close = getattr(self.engine, "close", None)
        if callable(close):
            close()

    def execute(self, plan: ResidentEpochPlan, snapshot: ResidentKVSnapshot | None = None,
                device_transfer: DeviceKVTransfer | None = None) -> ModelRunnerOutput:
        transfer = _Transfer.choose(snapshot, device_transfer)
        with _stage(EpochCommitState.PREPARED, "the plan was rejected before execution"):
            plan.validate()
            run = transfer.bind(self.engine)
        with _stage(EpochCommitState.EXECUTING, "the engine failed without proof of its commit state"):
            out = run(plan)
        if out.status != 0:
            raise ResidentEpochExecutionError(f"the device fell back with status {out.status}",
                                              commit_state=out.commit_state, status=out.status)
        if out.commit_state != EpochCommitState.COMMITTED:
            raise ResidentEpochExecutionError("the engine succeeded but did not commit",
                                              commit_state=out.commit_state)
        with _stage(EpochCommitState.COMMITTED, "the committed epoch's output is invalid"):
            transfer.check_proof(out)
            if set(out.token_ids) != set(plan.req_ids):
                raise ValueError(f"the engine answered for {sorted(out.token_ids)}, the plan asked for "
                                 f"{sorted(plan.req_ids)}")
            result = _device_result(plan, out, transfer)
            sampled = {rid: list(out.token_ids[rid]) for rid in plan.req_ids}
            result.validate_against(plan, sampled)
        req_ids = list(plan.req_ids)
        output = ModelRunnerOutput(req_ids=req_ids, req_id_to_index={rid: i for i, rid in enumerate(req_ids)},
                                   sampled_token_ids=[sampled[rid] for rid in req_ids])
        attach_result(output, result)
        return output


BACKEND_FACTORY_ENV = "VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY"


def load_backend_from_env() -> ResidentEpochBackend:
    """The backend over the engine that the factory named by
    VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY ("module:factory", e.g.
    "cruise_amd.sidecar_backend:create_sidecar_engine") returns."""
    target = os.getenv(BACKEND_FACTORY_ENV, "")
    module, sep, factory = target.partition(":")
    if not (module and sep and factory):
        raise RuntimeError(f"{BACKEND_FACTORY_ENV}={target!r}: expected module:factory naming the native engine")
    return ResidentEpochBackend(getattr(import_module(module), factory)())
