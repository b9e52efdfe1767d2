"""The scheduler <-> worker contract of a resident epoch.

Interface kept from src/vllm_ascend_resident_epoch/contract.py so that a
scheduler, worker or test written against the reference reads these objects
unchanged: the attribute names the plan and the result travel under
(contract.py:7-8), the three commit states (13-16), the execution error and
its ``input_preserving`` property (19-33), and the field names of the
request, plan and result records (36-136).  The same conditions are
rejected, always with ValueError (contract.py:75-112 for a plan, 138-214 for
a result).

The rules themselves are data here: each is a named predicate in an ordered
table, ``validate`` reports the first one broken as a ContractViolation (a
ValueError) whose ``rule`` attribute names it, and ``violations`` lists every
broken rule at once for diagnostics.
"""
from __future__ import annotations

from dataclasses import dataclass
from enum import IntEnum
from typing import Any, Callable, Iterator, Literal

from .version import PYTHON_CONTRACT_VERSION

PLAN_ATTR = "_ascend_resident_epoch_plan"
RESULT_ATTR = "_ascend_resident_epoch_result"
CONTRACT_VERSION = PYTHON_CONTRACT_VERSION
GRAPH_BATCH_SIZES = (1, 2, 4)
TRANSFER_MODES = ("none", "host_snapshot", "device_ipc")


class EpochCommitState(IntEnum):
    """How far an epoch got.  PREPARED: nothing reached the device, the host
    state is intact.  EXECUTING: the device may have run.  COMMITTED: the
    outputs were fetched and unpacked."""

    PREPARED = 0
    EXECUTING = 1
    COMMITTED = 2


class ResidentEpochExecutionError(RuntimeError):
    """An epoch failure and the commit state it reached.  Only a PREPARED
    failure leaves the host's copy of the requests valid, so only it may be
    replayed on the host."""

    def __init__(self, message: str, *, commit_state: EpochCommitState, status: int | None = None) -> None:
        super().__init__(message)
        self.commit_state = commit_state
        self.status = status

    @property
    def input_preserving(self) -> bool:
        return self.commit_state == EpochCommitState.PREPARED


class ContractViolation(ValueError):
    """A broken contract rule; ``rule`` is its name in the rule tables."""

    def __init__(self, rule: str, detail: str) -> None:
        super().__init__(f"[{rule}] {detail}")
        self.rule = rule


# A rule: (name, predicate that holds for a valid record, what a violation means).
Rule = tuple[str, Callable[..., bool], str]


def _broken(rules: tuple[Rule, ...], *record: Any) -> Iterator[ContractViolation]:
    """The violations of ``rules`` in table order.  A rule is only evaluated
    once every earlier one holds, so later predicates may rely on them; the
    iteration therefore stops at the first violation."""
    for name, holds, detail in rules:
        if not holds(*record):
            yield ContractViolation(name, detail)
            return


@dataclass(frozen=True)
class ResidentEpochRequest:
    """One resident row of a plan."""

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


def _distinct(values) -> bool:
    values = list(values)
    return len(set(values)) == len(values)


def _occupancy(plan: "ResidentEpochPlan") -> tuple[int, ...]:
    rows = {r.row for r in plan.requests}
    return tuple(int(row in rows) for row in range(plan.graph_batch_size))


PLAN_RULES: tuple[Rule, ...] = (
    ("contract-version", lambda p: p.version == CONTRACT_VERSION,
     f"the plan is not written for contract version {CONTRACT_VERSION}"),
    ("graph-batch", lambda p: p.graph_batch_size in GRAPH_BATCH_SIZES,
     f"graph batch size must be one of {GRAPH_BATCH_SIZES}"),
    ("request-count", lambda p: 0 < len(p.requests) <= p.graph_batch_size,
     "a plan carries between one request and one request per graph row"),
    ("mask-length", lambda p: len(p.active_mask) == p.graph_batch_size,
     "the active mask needs one entry per graph row"),
    ("mask-binary", lambda p: set(p.active_mask) <= {0, 1},
     "active mask entries are 0 or 1"),
    ("request-ids", lambda p: _distinct(p.req_ids),
     "a request appears at most once in a plan"),
    ("row-ids", lambda p: _distinct(r.row for r in p.requests),
     "two requests of a plan share a resident row"),
    ("generation-positive", lambda p: all(r.generation > 0 for r in p.requests),
     "resident generations start at 1"),
    ("generation-ids", lambda p: _distinct(r.generation for r in p.requests),
     "two requests of a plan share a generation"),
    ("row-range", lambda p: all(0 <= r.row < p.graph_batch_size for r in p.requests),
     "a request's row lies outside the graph"),
    ("length-position", lambda p: all(r.sequence_length == r.position + 1 for r in p.requests),
     "a request's sequence length must be its position plus one"),
    ("state-owner", lambda p: all(r.state_owner in ("host", "device") for r in p.requests),
     "state_owner is 'host' or 'device'"),
    ("import-owner", lambda p: all(r.state_owner == "host" for r in p.requests if r.kv_import_required),
     "only a request whose state the host still owns can have its KV imported"),
    ("capacity", lambda p: all(r.position + p.max_steps <= p.logical_capacity for r in p.requests),
     "position + max_steps exceeds the logical capacity of a row"),
    ("mask-rows", lambda p: _occupancy(p) == tuple(p.active_mask),
     "the active mask must mark exactly the rows the requests occupy"),
)


@dataclass(frozen=True)
class ResidentEpochPlan:
    """What one epoch must do: K = ``max_steps`` decoder steps over the
    requests, each on its own row of a ``graph_batch_size``-row graph."""

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

    def violations(self) -> list[ContractViolation]:
        return list(_broken(PLAN_RULES, self))

    def validate(self) -> None:
        for violation in _broken(PLAN_RULES, self):
            raise violation


def _steps_ok(res, plan, tokens) -> bool:
    return all(1 <= res.computed_steps[r.req_id] <= plan.max_steps for r in plan.requests)


def _counts_ok(res, plan, tokens) -> bool:
    return all(len(tokens[r.req_id]) == res.computed_steps[r.req_id] for r in plan.requests)


def _short_rows_end_at_eos(res, plan, tokens) -> bool:
    """A device row that ran fewer than K steps stopped because it sampled
    its EOS token."""
    for r in plan.requests:
        if res.computed_steps[r.req_id] < plan.max_steps:
            row_tokens = tokens[r.req_id]
            if not row_tokens or row_tokens[-1] != r.eos_token_id:
                return False
    return True


def _device(rule: Callable[..., bool]) -> Callable[..., bool]:
    return lambda res, plan, tokens: res.route != "device" or rule(res, plan, tokens)


def _fallback(rule: Callable[..., bool]) -> Callable[..., bool]:
    return lambda res, plan, tokens: res.route != "host_fallback" or rule(res, plan, tokens)


RESULT_RULES: tuple[Rule, ...] = (
    # what the result is about
    ("result-version", lambda res, plan, tok: res.version == plan.version,
     "the result answers a different contract version than the plan"),
    ("result-requests", lambda res, plan, tok: set(res.computed_steps) == set(plan.req_ids),
     "computed_steps must name exactly the plan's requests"),
    ("output-requests", lambda res, plan, tok: set(tok) == set(plan.req_ids),
     "the sampled tokens must name exactly the plan's requests"),
    # a device epoch: one complete, committed run of the planned rows
    ("device-status", _device(lambda res, plan, tok: res.status == 0),
     "a device epoch with a non-zero status cannot be committed"),
    ("device-committed", _device(lambda res, plan, tok: res.commit_state == EpochCommitState.COMMITTED),
     "a device epoch's result must be in the COMMITTED state"),
    ("device-round-trip", _device(lambda res, plan, tok: (res.feed_calls, res.fetch_calls) == (1, 1)),
     "a device epoch is one feed and one fetch"),
    ("device-generations", _device(lambda res, plan, tok: tuple(res.row_generations) == plan.row_generations),
     "the generations the device acknowledged differ from the plan's"),
    ("device-import", _device(lambda res, plan, tok: res.kv_imported
                              or not any(r.kv_import_required for r in plan.requests)),
     "the plan asked for a KV import that the device did not perform"),
    # an imported KV transfer must prove itself
    ("import-proof", lambda res, plan, tok: not res.kv_imported
     or (res.kv_import_checksum != 0 and res.transfer_mode in ("host_snapshot", "device_ipc")),
     "an imported KV transfer needs a non-zero checksum and a transfer mode"),
    ("snapshot-proof", lambda res, plan, tok: not (res.kv_imported and res.transfer_mode == "host_snapshot")
     or (res.kv_snapshot_checksum != 0 and res.kv_import_checksum == res.kv_snapshot_checksum),
     "the checksum of the imported KV differs from the host snapshot's"),
    ("transfer-without-import", lambda res, plan, tok: res.kv_imported or res.transfer_mode == "none",
     "a transfer mode is set although nothing was imported"),
    # a host fallback: nothing reached the device and the host may replay
    ("fallback-declared", _fallback(lambda res, plan, tok: res.fallback_safe),
     "a host fallback must be declared input-preserving"),
    ("fallback-prepared", _fallback(lambda res, plan, tok: res.commit_state == EpochCommitState.PREPARED),
     "a host fallback is only possible from the PREPARED state"),
    ("fallback-host-owned", _fallback(lambda res, plan, tok: plan.host_replay_safe),
     "a host fallback needs every request's state on the host"),
    ("fallback-no-dataflow", _fallback(lambda res, plan, tok: (res.feed_calls, res.fetch_calls) == (0, 0)),
     "a host fallback performed no feed or fetch"),
    # per request
    ("steps-range", _steps_ok, "each request runs between 1 and max_steps steps"),
    ("steps-tokens", _counts_ok, "each request samples one token per computed step"),
    ("fallback-one-step", _fallback(lambda res, plan, tok: set(res.computed_steps.values()) == {1}),
     "a host fallback keeps vLLM's one step per request"),
    ("short-row-eos", _device(_short_rows_end_at_eos),
     "a device row that stopped before K steps must end with its EOS token"),
    ("device-model-calls", _device(lambda res, plan, tok: res.model_calls == max(res.computed_steps.values())),
     "the device's decoder-step count must equal the longest row's steps"),
)


@dataclass(frozen=True)
class ResidentEpochResult:
    """What an epoch did, attached to the model-runner output."""

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

    @property
    def transfer_mode(self) -> str:
        """The transfer mode in effect: an import recorded without a mode
        came from a host snapshot."""
        if self.kv_imported and self.kv_transfer_mode == "none":
            return "host_snapshot"
        return self.kv_transfer_mode

    def violations(self, plan: ResidentEpochPlan, sampled_token_ids: dict[str, list[int]]) -> list[ContractViolation]:
        return list(_broken(RESULT_RULES, self, plan, sampled_token_ids))

    def validate_against(self, plan: ResidentEpochPlan, sampled_token_ids: dict[str, list[int]]) -> None:
        """Every rule an epoch result must satisfy before the scheduler
        advances its accounting; raises the first violation."""
        for violation in _broken(RESULT_RULES, self, plan, sampled_token_ids):
            raise violation


def attach_plan(scheduler_output: Any, plan: ResidentEpochPlan) -> None:
    plan.validate()
    setattr(scheduler_output, PLAN_ATTR, plan)


def get_plan(scheduler_output: Any) -> ResidentEpochPlan | None:
    return _typed_attr(scheduler_output, PLAN_ATTR, ResidentEpochPlan, "SchedulerOutput")


def attach_result(model_runner_output: Any, result: ResidentEpochResult) -> None:
    setattr(model_runner_output, RESULT_ATTR, result)


def get_result(model_runner_output: Any) -> ResidentEpochResult | None:
    return _typed_attr(model_runner_output, RESULT_ATTR, ResidentEpochResult, "ModelRunnerOutput")


def _typed_attr(holder: Any, attr: str, kind: type, holder_name: str):
    value = getattr(holder, attr, None)
    if value is not None and not isinstance(value, kind):
        raise TypeError(f"{holder_name}.{attr} holds a {type(value).__name__}, not a {kind.__name__}")
    return value
