"""Scheduler side of resident epochs: which requests run on the device, in
which resident row, under which generation, for how many steps (K).

Mirrors src/vllm_ascend_resident_epoch/scheduler.py:19-366 as a mixin over
any scheduler with vLLM v1's shape (``schedule``, ``update_from_output``,
``running``, ``waiting``, ``requests``, ``kv_cache_manager``, ...):

* ``ResidentEpochSchedulerMixin`` holds every rule of the reference
  scheduler -- row allocation (lowest free row, a fresh generation per
  request, rows freed when a request leaves the schedule), K selection (the
  largest of 1, 2, 4, 8 within the configured K and every request's remaining
  token budget), the eligibility and layout checks, isolation of host
  prefill from device-owned requests, and the accounting that advances
  ``num_computed_tokens`` by the steps the device actually ran.
* ``ResidentEpochScheduler`` is that mixin over vLLM's ``Scheduler`` when
  vLLM is installed.  Without vLLM the mixin is combined with any base of
  the same shape (the tests use a small in-memory one).
"""
from __future__ import annotations

from typing import Any

from .config import EPOCH_STEP_CHOICES, ResidentEpochConfig
from .contract import CONTRACT_VERSION, ResidentEpochPlan, ResidentEpochRequest, attach_plan, get_plan, get_result
from .eligibility import request_rejection_reason

GENERATION_LIMIT = 2**31
GRAPH_BATCH_SIZE = 4  # one B=4 graph serves every admitted batch size (scheduler.py:248-250)
NATIVE_MODEL = {"model_type": "qwen2", "num_hidden_layers": 28, "hidden_size": 3584, "vocab_size": 152064}


def epoch_steps_for(max_steps: int, remaining: list[int]) -> int:
    """K of the next epoch: the largest allowed step count that neither the
    configuration nor any request's remaining token budget forbids
    (scheduler.py:244-247)."""
    budget = min(max_steps, min(remaining))
    return max(k for k in EPOCH_STEP_CHOICES if k <= budget)


class ResidentEpochSchedulerMixin:
    """Resident-epoch planning over a vLLM-shaped scheduler (see module doc)."""

    def __init__(self, *args: Any, **kwargs: Any) -> None:
        super().__init__(*args, **kwargs)
        self._resident_epoch_config = ResidentEpochConfig.from_env()
        self._resident_epoch_last_rejection: str | None = None
        self._resident_epoch_last_plan: ResidentEpochPlan | None = None
        self._resident_epoch_last_result: Any | None = None
        self._resident_epoch_rows: dict[str, int] = {}
        self._resident_epoch_generations: dict[str, int] = {}
        self._resident_epoch_device_owned: set[str] = set()
        self._resident_epoch_next_generation = 1
        if self.vllm_config.speculative_config is not None:
            raise ValueError("resident epoch scheduler cannot be combined with speculative decoding")
        if self.scheduler_config.async_scheduling:
            raise ValueError("resident epoch scheduler requires synchronous scheduling")
        parallel = self.vllm_config.parallel_config
        if parallel.tensor_parallel_size != 1:
            raise ValueError("resident epoch scheduler currently requires tensor parallel size 1")
        if parallel.pipeline_parallel_size != 1:
            raise ValueError("resident epoch scheduler currently requires pipeline parallel size 1")
        reason = self._native_model_rejection_reason()
        if reason is not None:
            raise ValueError(f"resident epoch native graph mismatch: {reason}")

    # -- state -------------------------------------------------------------------
    def _ensure_test_config(self) -> ResidentEpochConfig:
        """Resident state for schedulers built without __init__ (tests build
        one with object.__new__ or by swapping __class__)."""
        if getattr(self, "_resident_epoch_config", None) is None:
            self._resident_epoch_config = ResidentEpochConfig()
            self._resident_epoch_last_rejection = None
        defaults = {
            "_resident_epoch_rows": dict,
            "_resident_epoch_generations": dict,
            "_resident_epoch_device_owned": set,
        }
        for name, make in defaults.items():
            if not hasattr(self, name):
                setattr(self, name, make())
        if not hasattr(self, "_resident_epoch_next_generation"):
            self._resident_epoch_next_generation = 1
        return self._resident_epoch_config

    def _assign_resident_rows(self, req_ids: tuple[str, ...]) -> None:
        """Free the rows of requests that left the schedule, then give each
        new request the lowest free row and the next generation
        (scheduler.py:63-86)."""
        keep = set(req_ids)
        for rid in [r for r in self._resident_epoch_rows if r not in keep]:
            del self._resident_epoch_rows[rid]
            del self._resident_epoch_generations[rid]
            self._resident_epoch_device_owned.discard(rid)
        taken = set(self._resident_epoch_rows.values())
        free = [row for row in range(self._resident_epoch_config.max_batch_size) if row not in taken]
        for rid in req_ids:
            if rid in self._resident_epoch_rows:
                continue
            if not free:
                raise RuntimeError("resident row allocator exhausted")
            if self._resident_epoch_next_generation >= GENERATION_LIMIT:
                raise RuntimeError("resident generation space exhausted")
            self._resident_epoch_rows[rid] = free.pop(0)
            self._resident_epoch_generations[rid] = self._resident_epoch_next_generation
            self._resident_epoch_next_generation += 1

    def _native_model_rejection_reason(self) -> str | None:
        hf = self.vllm_config.model_config.hf_config
        for field, expected in NATIVE_MODEL.items():
            actual = getattr(hf, field, None)
            if actual != expected:
                return f"{field}={actual!r}"
        return None

    # -- scheduling --------------------------------------------------------------
    def _host_isolation_reason(self, device_running: tuple[Any, ...]) -> str | None:
        """Why the host lane must run alone this step: a running host request
        the device cannot serve, or a prefill to admit (scheduler.py:102-128)."""
        if not device_running:
            return None
        host_running = [r for r in self.running if r not in device_running]
        if any(request_rejection_reason(r) is not None for r in host_running):
            return "unsupported-host-isolation"
        if any(r.num_computed_tokens < r.num_prompt_tokens for r in host_running):
            return "host-prefill-admission"
        waiting = list(self.waiting) + list(getattr(self, "skipped_waiting", ()))
        needs_prefill = any(r.num_prompt_tokens > 1 or request_rejection_reason(r) is not None for r in waiting)
        if needs_prefill and len(self.running) < self.max_num_running_reqs:
            return "host-prefill-admission"
        return None

    def _schedule_with_host_isolation(self) -> tuple[Any, tuple[str, ...], str | None]:
        """Run the base scheduler; when the host lane needs isolation, hide the
        device-owned requests from it for this one call (scheduler.py:130-161)."""
        device_running = tuple(r for r in self.running if r.request_id in self._resident_epoch_device_owned)
        reason = self._host_isolation_reason(device_running)
        if reason is None:
            return super().schedule(), (), None
        paused_ids = tuple(r.request_id for r in device_running)
        limit = self.max_num_running_reqs
        self.running[:] = [r for r in self.running if r not in device_running]
        self.max_num_running_reqs = limit - len(device_running)
        try:
            output = super().schedule()
        finally:
            self.running[:] = [*device_running, *self.running]
            self.max_num_running_reqs = limit
        scheduled = set(output.num_scheduled_tokens)
        if not scheduled:
            raise RuntimeError("isolated Host lane did not schedule a request")
        if scheduled & set(paused_ids):
            raise RuntimeError("isolated Host lane scheduled Device-owned state")
        return output, paused_ids, reason

    def schedule(self):
        self._ensure_test_config()
        if self.num_lookahead_tokens != 0:
            raise RuntimeError("resident epoch lookahead conflicts with another feature")
        output, paused_ids, isolation = self._schedule_with_host_isolation()
        plan, rejection = self._make_resident_epoch_plan(output)
        if plan is None:
            stranded = set(output.num_scheduled_tokens) & self._resident_epoch_device_owned
            if stranded:
                raise RuntimeError("refusing Host execution for Device-owned requests: " + ",".join(sorted(stranded)))
        if paused_ids:
            if plan is not None:
                raise RuntimeError("isolated Host lane created a resident plan")
            rejection = isolation
        self._resident_epoch_last_rejection = rejection
        self._resident_epoch_last_plan = plan
        self._resident_epoch_last_result = None
        if plan is not None:
            attach_plan(output, plan)
        return output

    def _schedule_rejection(self, output: Any, config: ResidentEpochConfig) -> str | None:
        """Batch-level reasons the scheduled step cannot be an epoch."""
        req_ids = tuple(output.num_scheduled_tokens)
        checks = (
            (lambda: not req_ids, "empty-schedule"),
            (lambda: len(req_ids) > config.max_batch_size, "batch-too-large"),
            (lambda: any(output.num_scheduled_tokens[r] != 1 for r in req_ids), "not-single-token-decode"),
            (lambda: bool(output.scheduled_spec_decode_tokens), "speculative-decode"),
            (lambda: bool(output.scheduled_encoder_inputs), "encoder-input"),
            (lambda: bool(output.preempted_req_ids), "preemption"),
            (lambda: self.connector is not None or self.ec_connector is not None, "cache-connector"),
            (lambda: self.block_size != config.block_size, "block-size"),
            (lambda: set(req_ids) != {r.request_id for r in self.running}, "partial-running-set"),
        )
        return next((reason for hit, reason in checks if hit()), None)

    def _request_rejection(self, request: Any, config: ResidentEpochConfig) -> str | None:
        """Per-request reasons (scheduler.py:224-241); None when eligible."""
        reason = request_rejection_reason(request)
        if reason is not None:
            return reason
        if request.num_prompt_tokens > config.logical_capacity:
            return "prompt-exceeds-resident-capacity"
        prefilled_on_host = request.num_prompt_tokens > 1
        if prefilled_on_host and request.num_output_tokens == 0:
            return "host-prefill-in-progress"
        if prefilled_on_host and request.request_id not in self._resident_epoch_device_owned:
            if len(self.kv_cache_manager.get_blocks(request.request_id).get_block_ids()) != 1:
                return "multiple-kv-cache-groups"
        if request.num_computed_tokens != request.num_tokens:
            return "computed-token-accounting"
        if request.max_tokens - request.num_output_tokens < 1:
            return "request-has-no-remaining-steps"
        return None

    def _make_resident_epoch_plan(self, output: Any) -> tuple[ResidentEpochPlan | None, str | None]:
        config = self._ensure_test_config()
        rejection = self._schedule_rejection(output, config)
        if rejection is not None:
            return None, rejection
        req_ids = tuple(output.num_scheduled_tokens)
        self._assign_resident_rows(req_ids)
        requests = [self.requests[rid] for rid in req_ids]
        for request in requests:
            rejection = self._request_rejection(request, config)
            if rejection is not None:
                return None, rejection
        steps = epoch_steps_for(config.max_steps, [r.max_tokens - r.num_output_tokens for r in requests])
        planned = []
        active = [0] * GRAPH_BATCH_SIZE
        for request in requests:
            rid = request.request_id
            row = self._resident_epoch_rows[rid]
            position = request.num_computed_tokens - 1
            if position < 0 or position + steps > config.logical_capacity:
                return None, "logical-capacity"
            groups = self.kv_cache_manager.get_blocks(rid).get_block_ids()
            if len(groups) != 1:
                return None, "multiple-kv-cache-groups"
            blocks = tuple(groups[0])
            if not blocks:
                return None, "missing-kv-block"
            owned = rid in self._resident_epoch_device_owned
            planned.append(
                ResidentEpochRequest(
                    req_id=rid,
                    row=row,
                    generation=self._resident_epoch_generations[rid],
                    token_id=int(request.all_token_ids[position]),
                    position=position,
                    sequence_length=position + 1,
                    eos_token_id=int(request.sampling_params.eos_token_id),
                    scheduler_block_ids=blocks,
                    device_block_ids=(row * config.blocks_per_request, row * config.blocks_per_request + 1),
                    state_owner="device" if owned else "host",
                    kv_import_required=request.num_prompt_tokens > 1 and not owned,
                )
            )
            active[row] = 1
        plan = ResidentEpochPlan(
            version=CONTRACT_VERSION,
            graph_batch_size=GRAPH_BATCH_SIZE,
            max_steps=steps,
            logical_capacity=config.logical_capacity,
            requests=tuple(planned),
            active_mask=tuple(active),
        )
        plan.validate()
        return plan, None

    # -- results -----------------------------------------------------------------
    def update_from_output(self, scheduler_output: Any, model_runner_output: Any):
        plan = get_plan(scheduler_output)
        result = get_result(model_runner_output)
        if plan is None:
            if result is not None:
                raise RuntimeError("resident epoch result has no scheduler plan")
            return super().update_from_output(scheduler_output, model_runner_output)
        if result is None:
            raise RuntimeError("resident epoch plan did not receive execution metadata")
        self._resident_epoch_last_result = result
        self._apply_resident_epoch_accounting(scheduler_output, model_runner_output, plan, result)
        return super().update_from_output(scheduler_output, model_runner_output)

    def _apply_resident_epoch_accounting(self, scheduler_output: Any, model_runner_output: Any,
                                         plan: ResidentEpochPlan, result: Any) -> None:
        """Advance each request by the steps the epoch ran beyond the one the
        base scheduler accounts for, then mark host-owned rows of a device
        epoch as device-owned (scheduler.py:330-366)."""
        index = model_runner_output.req_id_to_index
        sampled = {rid: list(model_runner_output.sampled_token_ids[index[rid]]) for rid in plan.req_ids}
        result.validate_against(plan, sampled)
        extras = {}
        for rid, steps in result.computed_steps.items():
            extra = steps - scheduler_output.num_scheduled_tokens[rid]
            if extra < 0:
                raise RuntimeError("resident epoch computed fewer than scheduled tokens")
            request = self.requests[rid]
            if request.num_computed_tokens + extra > request.num_tokens + len(sampled[rid]):
                raise RuntimeError("resident epoch would over-advance computed tokens")
            extras[rid] = extra
        for rid, extra in extras.items():
            self.requests[rid].num_computed_tokens += extra
        if result.route == "device":
            self._ensure_test_config()
            self._resident_epoch_device_owned.update(r.req_id for r in plan.requests if r.state_owner == "host")


try:  # pragma: no cover - vLLM is not part of every environment
    from vllm.v1.core.sched.scheduler import Scheduler as _VllmScheduler
except ImportError:  # pragma: no cover
    _VllmScheduler = None

if _VllmScheduler is not None:  # pragma: no cover

    class ResidentEpochScheduler(ResidentEpochSchedulerMixin, _VllmScheduler):
        """Scheduler extension for stateful fixed-shape resident epochs."""

else:
    ResidentEpochScheduler = None  # type: ignore[assignment]
