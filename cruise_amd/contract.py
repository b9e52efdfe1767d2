"""The scheduler <-> worker contract of a resident epoch.

Mirrors src/vllm_ascend_resident_epoch/contract.py: the plan the scheduler
attaches to its output (one request per resident row), the result the
worker attaches to the model-runner output, the three commit states and the
execution error that carries them.  Field names, validation rules and the
wording of the rejections are the reference's, so its scheduler, worker and
tests read these objects unchanged.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum
from typing import Any, Literal

from .version import PYTHON_CONTRACT_VERSION

PLAN_ATTR = "_ascend_resident_epoch_plan"
RESULT_ATTR = "_ascend_resident_epoch_result"
CONTRACT_VERSION = PYTHON_CONTRACT_VERSION


class EpochCommitState(IntEnum):
    """How far an epoch got (contract.py:13-16): PREPARED means nothing
    reached the device, EXECUTING that the device may have run, COMMITTED
    that the outputs were fetched and unpacked."""

    PREPARED = 0
    EXECUTING = 1
    COMMITTED = 2


class ResidentEpochExecutionError(RuntimeError):
    """An epoch failure together with the commit state it reached
    (contract.py:19-33).  Only a PREPARED failure leaves the host state
    intact, so only it may be replayed on the host."""

    def __init__(self, message: str, *, commit_state: EpochCommitState, status: int | None = None) -> None:
        super().__init__(message)
        self.commit_state = commit_state
        self.status = status

    @property
    def input_preserving(self) -> bool:
        return self.commit_state == EpochCommitState.PREPARED


def _check(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


@dataclass(frozen=True)
class ResidentEpochRequest:
    """One resident row of a plan (contract.py:36-48)."""

    req_id: str
    row: int
    generation: int
    token_id: int
    position: int
    sequence_length: int
    eos_token_id: int
    scheduler_block_ids: tuple[int, ...]
    device_block_ids: tuple[int, int]
    state_owner: Literal["host", "device"] = "host"
    kv_import_required: bool = False


@dataclass(frozen=True)
class ResidentEpochPlan:
    """What one epoch must do (contract.py:51-112)."""

    version: int
    graph_batch_size: Literal[1, 2, 4]
    max_steps: int
    logical_capacity: int
    requests: tuple[ResidentEpochRequest, ...]
    active_mask: tuple[int, ...]
    sampling_mode: int = 0
    graph_variant: int = 0

    @property
    def req_ids(self) -> tuple[str, ...]:
        return tuple(r.req_id for r in self.requests)

    @property
    def row_generations(self) -> tuple[int, ...]:
        """Generation per graph row, 0 for rows without a request."""
        by_row = {r.row: r.generation for r in self.requests}
        return tuple(by_row.get(row, 0) for row in range(self.graph_batch_size))

    @property
    def host_replay_safe(self) -> bool:
        return all(r.state_owner == "host" for r in self.requests)

    def validate(self) -> None:
        _check(self.version == CONTRACT_VERSION, f"unsupported resident epoch contract {self.version}")
        _check(self.graph_batch_size in (1, 2, 4), "graph batch size must be 1, 2, or 4")
        _check(1 <= len(self.requests) <= self.graph_batch_size, "request count does not fit the static graph")
        _check(len(self.active_mask) == self.graph_batch_size, "active mask does not match graph batch size")
        _check(all(v in (0, 1) for v in self.active_mask), "active mask must contain only zero or one")
        _check(len(set(self.req_ids)) == len(self.requests), "request IDs must be unique")
        rows = [r.row for r in self.requests]
        _check(len(set(rows)) == len(rows), "resident rows must be unique")
        gens = [r.generation for r in self.requests]
        _check(all(g > 0 for g in gens), "resident generations must be positive")
        _check(len(set(gens)) == len(gens), "resident generations must be unique")
        occupied = [0] * self.graph_batch_size
        for r in self.requests:
            _check(0 <= r.row < self.graph_batch_size, "resident row is outside the static graph")
            occupied[r.row] = 1
            _check(r.sequence_length == r.position + 1, "sequence length and position disagree")
            _check(r.state_owner in ("host", "device"), "resident request has an invalid state owner")
            _check(not r.kv_import_required or r.state_owner == "host", "KV import requires Host-owned request state")
            _check(r.position + self.max_steps <= self.logical_capacity, "epoch exceeds logical capacity")
        _check(tuple(occupied) == tuple(self.active_mask), "active mask does not match resident rows")


@dataclass(frozen=True)
class ResidentEpochResult:
    """What an epoch did (contract.py:115-214)."""

    version: int
    route: Literal["device", "host_fallback"]
    status: int
    model_calls: int
    computed_steps: dict[str, int]
    row_generations: tuple[int, ...] = ()
    commit_state: EpochCommitState = EpochCommitState.COMMITTED
    fallback_safe: bool = False
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
    kv_snapshot_checksum: int = 0
    kv_transfer_mode: Literal["none", "host_snapshot", "device_ipc"] = "none"

    def validate_against(self, plan: ResidentEpochPlan, sampled_token_ids: dict[str, list[int]]) -> None:
        """Every rule a committed or host-replayed epoch must satisfy before
        the scheduler advances its accounting (contract.py:138-214)."""
        device = self.route == "device"
        fallback = self.route == "host_fallback"
        _check(self.version == plan.version, "resident epoch result version mismatch")
        _check(set(self.computed_steps) == set(plan.req_ids), "resident epoch result request set mismatch")
        _check(set(sampled_token_ids) == set(plan.req_ids), "resident epoch output request set mismatch")
        if device:
            _check(self.status == 0, "failed device execution cannot be committed")
            _check(self.commit_state == EpochCommitState.COMMITTED, "device execution result is not committed")
            _check(self.feed_calls == 1 and self.fetch_calls == 1, "device epoch must use exactly one Feed and one Fetch")
            _check(self.row_generations == plan.row_generations, "device resident generations disagree with the plan")
            importing = any(r.kv_import_required for r in plan.requests)
            _check(not importing or self.kv_imported, "device result did not commit the requested KV import")
        # A result that imported without naming a mode came from a host snapshot.
        mode = "host_snapshot" if self.kv_imported and self.kv_transfer_mode == "none" else self.kv_transfer_mode
        if self.kv_imported:
            _check(
                self.kv_import_checksum != 0 and mode in ("host_snapshot", "device_ipc"),
                "device result did not prove an imported KV transfer",
            )
            if mode == "host_snapshot":
                _check(
                    self.kv_snapshot_checksum != 0 and self.kv_import_checksum == self.kv_snapshot_checksum,
                    "device result did not prove equivalent imported KV from the Host snapshot",
                )
        else:
            _check(mode == "none", "KV transfer mode is set without an import")
        if fallback:
            _check(self.fallback_safe, "host fallback must be declared input-preserving")
            _check(self.commit_state == EpochCommitState.PREPARED, "host fallback requires a prepared device state")
            _check(plan.host_replay_safe, "Host no longer owns every request state")
            _check(self.feed_calls == 0 and self.fetch_calls == 0, "Host fallback result cannot claim DataFlow calls")
        for r in plan.requests:
            steps = self.computed_steps[r.req_id]
            tokens = sampled_token_ids[r.req_id]
            _check(1 <= steps <= plan.max_steps, "computed step count is outside the epoch")
            _check(len(tokens) == steps, "sampled token count and computed steps disagree")
            if fallback:
                _check(steps == 1, "host fallback must retain one-step vLLM semantics")
            if device and steps < plan.max_steps:
                _check(bool(tokens) and tokens[-1] == r.eos_token_id, "a short device epoch must terminate at EOS")
        if device:
            _check(
                self.model_calls == max(self.computed_steps.values()),
                "device model-call count disagrees with executed steps",
            )


def attach_plan(scheduler_output: Any, plan: ResidentEpochPlan) -> None:
    plan.validate()
    setattr(scheduler_output, PLAN_ATTR, plan)


def get_plan(scheduler_output: Any) -> ResidentEpochPlan | None:
    plan = getattr(scheduler_output, PLAN_ATTR, None)
    if plan is not None and not isinstance(plan, ResidentEpochPlan):
        raise TypeError("invalid resident epoch plan attached to SchedulerOutput")
    return plan


def attach_result(model_runner_output: Any, result: ResidentEpochResult) -> None:
    setattr(model_runner_output, RESULT_ATTR, result)


def get_result(model_runner_output: Any) -> ResidentEpochResult | None:
    result = getattr(model_runner_output, RESULT_ATTR, None)
    if result is not None and not isinstance(result, ResidentEpochResult):
        raise TypeError("invalid resident epoch result attached to ModelRunnerOutput")
    return result
