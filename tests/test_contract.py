"""The scheduler/worker contract (cruise_amd.contract), restating the rules
the reference's tests/test_contract.py pins: short device epochs end at EOS,
host fallback keeps one-step accounting, only COMMITTED device results are
accepted, only PREPARED errors preserve the input, KV import needs host
ownership and a checksum proof; plus the plan validation rules of
contract.py:77-112 one by one.  Every violation names its rule, and the
tables below break every rule of both rule tables at least once."""
from __future__ import annotations

from dataclasses import replace

import pytest

from cruise_amd.contract import (
    CONTRACT_VERSION,
    PLAN_RULES,
    RESULT_RULES,
    ContractViolation,
    EpochCommitState,
    ResidentEpochExecutionError,
    ResidentEpochPlan,
    ResidentEpochRequest,
    ResidentEpochResult,
    attach_plan,
    attach_result,
    get_plan,
    get_result,
)


def base_request(**kw):
    fields = dict(req_id="r0", row=0, generation=1, token_id=1, position=0, sequence_length=1, eos_token_id=9,
                  scheduler_block_ids=(17,), device_block_ids=(0, 1))
    fields.update(kw)
    return ResidentEpochRequest(**fields)


def base_plan(*requests, batch=1, steps=4, capacity=8):
    requests = requests or (base_request(),)
    mask = [0] * batch
    for r in requests:
        mask[r.row] = 1
    return ResidentEpochPlan(CONTRACT_VERSION, batch, steps, capacity, tuple(requests), tuple(mask))


def device_result(plan, steps, **kw):
    return ResidentEpochResult(version=CONTRACT_VERSION, route="device", status=0, model_calls=max(steps.values()),
                               computed_steps=steps, row_generations=plan.row_generations, **kw)


def fallback_result(**kw):
    return ResidentEpochResult(version=CONTRACT_VERSION, route="host_fallback", status=0, model_calls=1,
                               computed_steps={"r0": 1}, commit_state=EpochCommitState.PREPARED, fallback_safe=True,
                               feed_calls=0, fetch_calls=0, **kw)


def broken(rule):
    """Expect a ContractViolation of ``rule`` (a ValueError)."""
    class Check:
        def __enter__(self):
            self.ctx = pytest.raises(ContractViolation)
            self.info = self.ctx.__enter__()
            return self.info

        def __exit__(self, *exc):
            handled = self.ctx.__exit__(*exc)
            assert isinstance(self.info.value, ValueError)
            assert self.info.value.rule == rule, str(self.info.value)
            return handled
    return Check()


def test_short_device_result_requires_eos():
    plan = base_plan()
    result = device_result(plan, {"r0": 2})
    with broken("short-row-eos"):
        result.validate_against(plan, {"r0": [3, 4]})
    result.validate_against(plan, {"r0": [3, 9]})


def test_full_device_epoch_needs_no_eos():
    plan = base_plan()
    device_result(plan, {"r0": 4}).validate_against(plan, {"r0": [2, 3, 4, 5]})


def test_host_fallback_keeps_one_step_accounting():
    fallback_result().validate_against(base_plan(), {"r0": [3]})
    with broken("fallback-one-step"):
        replace(fallback_result(), computed_steps={"r0": 2}, model_calls=2).validate_against(base_plan(), {"r0": [3, 4]})


@pytest.mark.parametrize("state", [EpochCommitState.PREPARED, EpochCommitState.EXECUTING])
def test_device_result_requires_committed_state(state):
    plan = base_plan()
    with broken("device-committed"):
        device_result(plan, {"r0": 4}, commit_state=state).validate_against(plan, {"r0": [2, 3, 4, 5]})


def test_host_fallback_rejects_device_owned_request():
    plan = base_plan(base_request(state_owner="device"))
    with broken("fallback-host-owned"):
        fallback_result().validate_against(plan, {"r0": [3]})


def test_only_prepared_execution_error_is_input_preserving():
    states = {s: ResidentEpochExecutionError("x", commit_state=s).input_preserving for s in EpochCommitState}
    assert states == {EpochCommitState.PREPARED: True, EpochCommitState.EXECUTING: False,
                      EpochCommitState.COMMITTED: False}


def test_kv_import_requires_host_ownership_and_commit_acknowledgement():
    plan = base_plan(base_request(kv_import_required=True))
    plan.validate()
    tokens = {"r0": [2, 3, 4, 5]}
    plain = device_result(plan, {"r0": 4})
    with broken("device-import"):
        plain.validate_against(plan, tokens)
    proven = replace(plain, kv_imported=True, kv_import_checksum=123, kv_snapshot_checksum=123)
    assert proven.transfer_mode == "host_snapshot"  # an import without a mode came from a snapshot
    proven.validate_against(plan, tokens)
    with broken("snapshot-proof"):
        replace(proven, kv_import_checksum=124).validate_against(plan, tokens)
    with broken("snapshot-proof"):
        replace(proven, kv_snapshot_checksum=0, kv_import_checksum=0x55).validate_against(plan, tokens)
    # a device-IPC import needs only a non-zero import checksum
    replace(plain, kv_imported=True, kv_import_checksum=5, kv_transfer_mode="device_ipc").validate_against(plan, tokens)
    with broken("import-proof"):
        replace(plain, kv_imported=True, kv_import_checksum=0, kv_transfer_mode="device_ipc").validate_against(plan, tokens)
    with broken("transfer-without-import"):
        replace(plain, kv_transfer_mode="device_ipc").validate_against(base_plan(), tokens)
    with broken("import-owner"):
        base_plan(base_request(kv_import_required=True, state_owner="device")).validate()


RESULT_CASES = [
    ({"status": 3}, "device-status"),
    ({"feed_calls": 2}, "device-round-trip"),
    ({"row_generations": (5,)}, "device-generations"),
    ({"model_calls": 3}, "device-model-calls"),
    ({"version": CONTRACT_VERSION + 1}, "result-version"),
    ({"computed_steps": {"r0": 9}}, "steps-range"),
    ({"computed_steps": {"r0": 0}}, "steps-range"),
    ({"computed_steps": {"x": 4}}, "result-requests"),
    ({"commit_state": EpochCommitState.EXECUTING}, "device-committed"),
]


@pytest.mark.parametrize(("result_kw", "rule"), RESULT_CASES)
def test_device_result_rules(result_kw, rule):
    plan = base_plan()
    result = replace(device_result(plan, {"r0": 4}), **result_kw)
    with broken(rule):
        result.validate_against(plan, {"r0": [2, 3, 4, 5]})
    assert [v.rule for v in result.violations(plan, {"r0": [2, 3, 4, 5]})] == [rule]


FALLBACK_CASES = [
    ({"fallback_safe": False}, "fallback-declared"),
    ({"commit_state": EpochCommitState.EXECUTING}, "fallback-prepared"),
    ({"feed_calls": 1}, "fallback-no-dataflow"),
]


@pytest.mark.parametrize(("result_kw", "rule"), FALLBACK_CASES)
def test_host_fallback_rules(result_kw, rule):
    with broken(rule):
        replace(fallback_result(), **result_kw).validate_against(base_plan(), {"r0": [3]})


def test_sampled_tokens_must_match_steps():
    plan = base_plan()
    with broken("steps-tokens"):
        device_result(plan, {"r0": 4}).validate_against(plan, {"r0": [2, 3]})
    with broken("output-requests"):
        device_result(plan, {"r0": 4}).validate_against(plan, {})


PLAN_CASES = [
    (lambda: replace(base_plan(), version=2), "contract-version"),
    (lambda: base_plan(batch=3), "graph-batch"),
    (lambda: replace(base_plan(), active_mask=(1, 0)), "mask-length"),
    (lambda: replace(base_plan(batch=2), active_mask=(1, 2)), "mask-binary"),
    (lambda: ResidentEpochPlan(CONTRACT_VERSION, 2, 4, 8, (base_request(), base_request(row=1, generation=2)), (1, 1)),
     "request-ids"),
    (lambda: ResidentEpochPlan(CONTRACT_VERSION, 2, 4, 8,
                               (base_request(), base_request(req_id="r1", generation=2)), (1, 1)), "row-ids"),
    (lambda: base_plan(base_request(generation=0)), "generation-positive"),
    (lambda: ResidentEpochPlan(CONTRACT_VERSION, 2, 4, 8, (base_request(), base_request(req_id="r1", row=1)), (1, 1)),
     "generation-ids"),
    (lambda: ResidentEpochPlan(CONTRACT_VERSION, 1, 4, 8, (base_request(row=1),), (1,)), "row-range"),
    (lambda: base_plan(base_request(sequence_length=3)), "length-position"),
    (lambda: base_plan(base_request(state_owner="gpu")), "state-owner"),
    (lambda: base_plan(base_request(kv_import_required=True, state_owner="device")), "import-owner"),
    (lambda: base_plan(base_request(position=5, sequence_length=6)), "capacity"),
    (lambda: replace(base_plan(base_request(), batch=2), active_mask=(0, 1)), "mask-rows"),
    (lambda: ResidentEpochPlan(CONTRACT_VERSION, 1, 4, 8, (), (0,)), "request-count"),
]


@pytest.mark.parametrize(("plan_fn", "rule"), PLAN_CASES)
def test_plan_validation_rules(plan_fn, rule):
    with broken(rule):
        plan_fn().validate()


def test_capacity_bound_is_inclusive():
    """pos + K == capacity still fits (contract.py:109): the last step writes
    slot capacity-1."""
    base_plan(base_request(position=4, sequence_length=5), steps=4, capacity=8).validate()


def test_every_rule_is_exercised():
    plan_rules = {rule for _, rule in PLAN_CASES}
    result_rules = ({rule for _, rule in RESULT_CASES} | {rule for _, rule in FALLBACK_CASES}
                    | {"short-row-eos", "fallback-one-step", "fallback-host-owned", "device-import", "snapshot-proof",
                       "import-proof", "transfer-without-import", "steps-tokens", "output-requests"})
    assert plan_rules == {name for name, _, _ in PLAN_RULES}
    assert result_rules == {name for name, _, _ in RESULT_RULES}


def test_row_generations_and_attachment():
    plan = base_plan(base_request(row=2, generation=7), batch=4)
    assert plan.row_generations == (0, 0, 7, 0)
    holder = type("Out", (), {})()
    attach_plan(holder, plan)
    assert get_plan(holder) is plan
    result = device_result(plan, {"r0": 4})
    attach_result(holder, result)
    assert get_result(holder) is result
    holder._ascend_resident_epoch_plan = "x"
    with pytest.raises(TypeError):
        get_plan(holder)
    with broken("generation-positive"):
        attach_plan(type("Out", (), {})(), base_plan(base_request(generation=-1)))
