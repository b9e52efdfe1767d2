"""Scheduler side of resident epochs: which requests an epoch serves, on which
graph row, under which generation, for how many steps.

Behaviour kept from src/vllm_ascend_resident_epoch/scheduler.py, because a
scheduler that replaces it must plan identically:

* rows and generations (scheduler.py:63-86): a request keeps its row while it
  stays scheduled; a new request takes the lowest free row and the next
  generation (1, 2, 3, ... below 2^31); a request that leaves the schedule
  frees its row and its device ownership;
* K (244-247): the largest of 1, 2, 4, 8 within the configured K and every
  request's remaining token budget;
* the rejection reasons and their precedence (194-241, 250-266), reported
  through ``_resident_epoch_last_rejection``;
* host isolation (102-161): while the device owns requests, a host request
  that needs prefill or cannot run on the device is scheduled alone, with
  the device-owned requests hidden from the base scheduler;
* accounting (330-366): a committed epoch advances each request's computed
  tokens by the steps beyond the one the base scheduler accounts for, and a
  device epoch moves host-owned requests to device ownership.

The structure is this module's own.  ``ResidentRowTable`` is the row and
generation bookkeeping on its own; ``plan_epoch`` is a function from the
scheduler's view and that table to a ``PlanDecision``; ``host_lane_reason``
and ``hide_device_rows`` are the isolation rule and mechanism; and
``advance_computed_tokens`` is the accounting.  ``ResidentEpochSchedulerMixin``
only wires them into a scheduler of vLLM v1's shape (``schedule``,
``update_from_output``, ``running``, ``waiting``, ``requests``,
``kv_cache_manager``, ...); ``ResidentEpochScheduler`` is that mixin over
vLLM's ``Scheduler`` when vLLM is installed.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from typing import Any, Iterator

from .config import GRAPH_ROWS, ResidentEpochConfig, epoch_steps_within
from .contract import CONTRACT_VERSION, ResidentEpochPlan, ResidentEpochRequest, attach_plan, get_plan, get_result
from .eligibility import request_rejection_reason

GENERATION_LIMIT = 2**31
# the model the native graph is built for
NATIVE_MODEL = {"model_type": "qwen2", "num_hidden_layers": 28, "hidden_size": 3584, "vocab_size": 152064}


def epoch_steps_for(max_steps: int, remaining: list[int]) -> int:
    """K of the next epoch for requests with ``remaining`` token budgets."""
    return epoch_steps_within(min(max_steps, *remaining))


# ---------------------------------------------------------------------------
# rows and generations
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Seat:
    row: int
    generation: int


class ResidentRowTable:
    """Which request sits on which graph row under which generation, and
    whose decode state the device owns."""

    def __init__(self, rows: int = GRAPH_ROWS, first_generation: int = 1) -> None:
        self.rows = rows
        self.seats: dict[str, Seat] = {}
        self.device_owned: set[str] = set()
        self.next_generation = first_generation

    def free_rows(self) -> list[int]:
        taken = {seat.row for seat in self.seats.values()}
        return [row for row in range(self.rows) if row not in taken]

    def release(self, req_id: str) -> None:
        self.seats.pop(req_id, None)
        self.device_owned.discard(req_id)

    def admit(self, req_id: str) -> Seat:
        free = self.free_rows()
        if not free:
            raise RuntimeError(f"no free resident row for {req_id}: all {self.rows} rows are taken (allocator "
                               "exhausted)")
        if self.next_generation >= GENERATION_LIMIT:
            raise RuntimeError("the resident generation space exhausted: generations are positive int32")
        seat = Seat(free[0], self.next_generation)
        self.seats[req_id] = seat
        self.next_generation += 1
        return seat

    def seat_exactly(self, req_ids: tuple[str, ...]) -> None:
        """Seat exactly ``req_ids``: free everyone else's row first, then
        admit newcomers in order."""
        for req_id in [r for r in self.seats if r not in set(req_ids)]:
            self.release(req_id)
        for req_id in req_ids:
            if req_id not in self.seats:
                self.admit(req_id)

    def owner(self, req_id: str) -> str:
        return "device" if req_id in self.device_owned else "host"


# ---------------------------------------------------------------------------
# planning
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class PlanDecision:
    plan: ResidentEpochPlan | None
    reason: str | None

    @classmethod
    def reject(cls, reason: str) -> "PlanDecision":
        return cls(None, reason)


def _block_groups(sched: Any, req_id: str):
    return sched.kv_cache_manager.get_blocks(req_id).get_block_ids()


def _batch_reason(sched: Any, output: Any, config: ResidentEpochConfig) -> str | None:
    """Why the scheduled step as a whole cannot be an epoch."""
    counts = output.num_scheduled_tokens
    if not counts:
        return "empty-schedule"
    if len(counts) > config.max_batch_size:
        return "batch-too-large"
    if set(counts.values()) != {1}:
        return "not-single-token-decode"
    for attribute, reason in (("scheduled_spec_decode_tokens", "speculative-decode"),
                              ("scheduled_encoder_inputs", "encoder-input"), ("preempted_req_ids", "preemption")):
        if getattr(output, attribute):
            return reason
    if sched.connector is not None or sched.ec_connector is not None:
        return "cache-connector"
    if sched.block_size != config.block_size:
        return "block-size"
    if set(counts) != {r.request_id for r in sched.running}:
        return "partial-running-set"
    return None


def _request_reason(sched: Any, request: Any, table: ResidentRowTable, config: ResidentEpochConfig) -> str | None:
    """Why one request cannot join the epoch."""
    reason = request_rejection_reason(request)
    if reason is not None:
        return reason
    if request.num_prompt_tokens > config.logical_capacity:
        return "prompt-exceeds-resident-capacity"
    host_prefilled = request.num_prompt_tokens > 1
    if host_prefilled and request.num_output_tokens == 0:
        return "host-prefill-in-progress"
    if (host_prefilled and request.request_id not in table.device_owned
            and len(_block_groups(sched, request.request_id)) != 1):
        return "multiple-kv-cache-groups"
    if request.num_computed_tokens != request.num_tokens:
        return "computed-token-accounting"
    if request.max_tokens - request.num_output_tokens < 1:
        return "request-has-no-remaining-steps"
    return None


def plan_epoch(sched: Any, output: Any, table: ResidentRowTable, config: ResidentEpochConfig) -> PlanDecision:
    """The epoch for the base scheduler's ``output``, or why there is none.
    Rows are (re)assigned as soon as the batch as a whole qualifies, before
    the per-request checks, so a request keeps its row across a rejected
    step."""
    reason = _batch_reason(sched, output, config)
    if reason is not None:
        return PlanDecision.reject(reason)
    req_ids = tuple(output.num_scheduled_tokens)
    table.seat_exactly(req_ids)
    requests = [sched.requests[rid] for rid in req_ids]
    for request in requests:
        reason = _request_reason(sched, request, table, config)
        if reason is not None:
            return PlanDecision.reject(reason)
    steps = config.epoch_steps(min(r.max_tokens - r.num_output_tokens for r in requests))

    rows = []
    for request in requests:
        rid = request.request_id
        position = request.num_computed_tokens - 1
        if position < 0 or position + steps > config.logical_capacity:
            return PlanDecision.reject("logical-capacity")
        groups = _block_groups(sched, rid)
        if len(groups) != 1:
            return PlanDecision.reject("multiple-kv-cache-groups")
        if not groups[0]:
            return PlanDecision.reject("missing-kv-block")
        seat = table.seats[rid]
        owner = table.owner(rid)
        rows.append(ResidentEpochRequest(
            req_id=rid, row=seat.row, generation=seat.generation, token_id=int(request.all_token_ids[position]),
            position=position, sequence_length=position + 1,
            eos_token_id=int(request.sampling_params.eos_token_id), scheduler_block_ids=tuple(groups[0]),
            device_block_ids=config.row_blocks(seat.row), state_owner=owner,
            kv_import_required=request.num_prompt_tokens > 1 and owner == "host",
        ))
    # One 4-row graph serves every admitted batch size: a graph per size
    # would hold another copy of the weights.
    occupied = {r.row for r in rows}
    plan = ResidentEpochPlan(
        version=CONTRACT_VERSION, graph_batch_size=GRAPH_ROWS, max_steps=steps,
        logical_capacity=config.logical_capacity, requests=tuple(rows),
        active_mask=tuple(int(row in occupied) for row in range(GRAPH_ROWS)),
    )
    plan.validate()
    return PlanDecision(plan, None)


# ---------------------------------------------------------------------------
# host isolation
# ---------------------------------------------------------------------------
def host_lane_reason(sched: Any, device_running: list[Any]) -> str | None:
    """Why host work must be scheduled alone this step, or None.  Only
    relevant while the device owns running requests."""
    if not device_running:
        return None
    host_running = [r for r in sched.running if r not in device_running]
    if any(request_rejection_reason(r) is not None for r in host_running):
        return "unsupported-host-isolation"
    if any(r.num_computed_tokens < r.num_prompt_tokens for r in host_running):
        return "host-prefill-admission"
    waiting = [*sched.waiting, *getattr(sched, "skipped_waiting", ())]
    wants_host = any(r.num_prompt_tokens > 1 or request_rejection_reason(r) is not None for r in waiting)
    if wants_host and len(sched.running) < sched.max_num_running_reqs:
        return "host-prefill-admission"
    return None


@contextmanager
def hide_device_rows(sched: Any, device_running: list[Any]) -> Iterator[None]:
    """Within the block the base scheduler sees neither the device-owned
    running requests nor the running slots they hold."""
    limit = sched.max_num_running_reqs
    sched.running[:] = [r for r in sched.running if r not in device_running]
    sched.max_num_running_reqs = limit - len(device_running)
    try:
        yield
    finally:
        sched.running[:] = [*device_running, *sched.running]
        sched.max_num_running_reqs = limit


# ---------------------------------------------------------------------------
# accounting
# ---------------------------------------------------------------------------
def advance_computed_tokens(sched: Any, scheduler_output: Any, model_runner_output: Any,
                            plan: ResidentEpochPlan, result: Any) -> None:
    """Validate the result against the plan, then move each request's
    computed-token count forward by the steps the epoch ran beyond the one
    the base scheduler's own update accounts for."""
    index = model_runner_output.req_id_to_index
    sampled = {rid: list(model_runner_output.sampled_token_ids[index[rid]]) for rid in plan.req_ids}
    result.validate_against(plan, sampled)
    extra = {}
    for rid, steps in result.computed_steps.items():
        extra[rid] = steps - scheduler_output.num_scheduled_tokens[rid]
        if extra[rid] < 0:
            raise RuntimeError(f"the epoch computed {steps} tokens for {rid}, fewer than were scheduled")
        request = sched.requests[rid]
        if request.num_computed_tokens + extra[rid] > request.num_tokens + len(sampled[rid]):
            raise RuntimeError(f"the epoch would over-advance computed tokens for {rid} past its sampled tokens")
    for rid, n in extra.items():
        sched.requests[rid].num_computed_tokens += n


# ---------------------------------------------------------------------------
# the scheduler
# ---------------------------------------------------------------------------
def unsupported_engine_reason(sched: Any) -> str | None:
    """Why this serving configuration cannot host resident epochs."""
    vllm = sched.vllm_config
    if vllm.speculative_config is not None:
        return "speculative decoding is enabled"
    if sched.scheduler_config.async_scheduling:
        return "asynchronous scheduling is enabled; epochs need synchronous scheduling"
    parallel = vllm.parallel_config
    if (parallel.tensor_parallel_size, parallel.pipeline_parallel_size) != (1, 1):
        return "tensor and pipeline parallel size must both be 1"
    hf = vllm.model_config.hf_config
    for name, expected in NATIVE_MODEL.items():
        if getattr(hf, name, None) != expected:
            return f"the native graph is built for {name}={expected!r}, the model has {getattr(hf, name, None)!r}"
    return None


class ResidentEpochSchedulerMixin:
    """Resident-epoch planning over a scheduler of vLLM v1's shape."""

    def __init__(self, *args: Any, **kwargs: Any) -> None:
        super().__init__(*args, **kwargs)
        self._resident_epoch_config = ResidentEpochConfig.from_env()
        self._resident_table = ResidentRowTable(self._resident_epoch_config.max_batch_size)
        self._resident_epoch_last_rejection: str | None = None
        self._resident_epoch_last_plan: ResidentEpochPlan | None = None
        self._resident_epoch_last_result: Any | None = None
        reason = unsupported_engine_reason(self)
        if reason is not None:
            raise ValueError(f"resident epoch scheduler: {reason}")

    def _resident_state(self) -> tuple[ResidentEpochConfig, ResidentRowTable]:
        """The configuration and row table; a scheduler assembled without
        this class's __init__ (as some tests do) gets defaults."""
        if getattr(self, "_resident_epoch_config", None) is None:
            self._resident_epoch_config = ResidentEpochConfig()
            self._resident_epoch_last_rejection = None
        if getattr(self, "_resident_table", None) is None:
            self._resident_table = ResidentRowTable(self._resident_epoch_config.max_batch_size)
        return self._resident_epoch_config, self._resident_table

    @property
    def _resident_epoch_device_owned(self) -> set[str]:
        return self._resident_state()[1].device_owned

    def schedule(self):
        config, table = self._resident_state()
        if self.num_lookahead_tokens != 0:
            raise RuntimeError("lookahead tokens cannot be combined with resident epochs")
        device_running = [r for r in self.running if r.request_id in table.device_owned]
        isolation = host_lane_reason(self, device_running)
        if isolation is None:
            output = super().schedule()
        else:
            with hide_device_rows(self, device_running):
                output = super().schedule()
            lane = set(output.num_scheduled_tokens)
            if not lane:
                raise RuntimeError("the isolated host lane scheduled nothing")
            if lane & {r.request_id for r in device_running}:
                raise RuntimeError("the isolated host lane scheduled a device-owned request")

        decision = plan_epoch(self, output, table, config)
        if decision.plan is None:
            stranded = set(output.num_scheduled_tokens) & table.device_owned
            if stranded:
                raise RuntimeError("device-owned requests cannot run on the host: " + ",".join(sorted(stranded)))
        elif isolation is not None:
            raise RuntimeError("the isolated host lane produced a resident plan")
        self._resident_epoch_last_rejection = isolation if isolation is not None else decision.reason
        self._resident_epoch_last_plan = decision.plan
        self._resident_epoch_last_result = None
        if decision.plan is not None:
            attach_plan(output, decision.plan)
        return output

    def update_from_output(self, scheduler_output: Any, model_runner_output: Any):
        plan = get_plan(scheduler_output)
        result = get_result(model_runner_output)
        if plan is None and result is not None:
            raise RuntimeError("an epoch result arrived for a step without a resident plan")
        if plan is not None:
            if result is None:
                raise RuntimeError("a resident plan's step returned no epoch result")
            self._resident_epoch_last_result = result
            self._apply_resident_epoch_accounting(scheduler_output, model_runner_output, plan, result)
        return super().update_from_output(scheduler_output, model_runner_output)

    def _apply_resident_epoch_accounting(self, scheduler_output: Any, model_runner_output: Any,
                                         plan: ResidentEpochPlan, result: Any) -> None:
        advance_computed_tokens(self, scheduler_output, model_runner_output, plan, result)
        if result.route == "device":
            table = self._resident_state()[1]
            table.device_owned.update(r.req_id for r in plan.requests if r.state_owner == "host")


try:  # pragma: no cover - vLLM is not part of every environment
    from vllm.v1.core.sched.scheduler import Scheduler as _VllmScheduler
except ImportError:  # pragma: no cover
    _VllmScheduler = None

if _VllmScheduler is not None:  # pragma: no cover

    class ResidentEpochScheduler(ResidentEpochSchedulerMixin, _VllmScheduler):
        """vLLM's scheduler with resident epochs."""

else:
    ResidentEpochScheduler = None  # type: ignore[assignment]
