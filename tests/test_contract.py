"""The scheduler/worker contract (cruise_amd.contract), restating the rules
the reference's tests/test_contract.py pins: short device epochs end at EOS,
host fallback keeps one-step accounting, only COMMITTED device results are
accepted, only PREPARED errors preserve the input, KV import needs host
ownership and a checksum proof; plus the plan validation rules of
contract.py:77-112 one by one."""
from __future__ import annotations

from dataclasses import replace

import pytest

from cruise_amd.contract import (
    CONTRACT_VERSION,
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


def test_short_device_result_requires_eos():
    plan = base_plan()
    result = device_result(plan, {"r0": 2})
    with pytest.raises(ValueError, match="terminate at EOS"):
        result.validate_against(plan, {"r0": [3, 4]})
    result.validate_against(plan, {"r0": [3, 9]})


def test_full_device_epoch_needs_no_eos():
    plan = base_plan()
    device_result(plan, {"r0": 4}).validate_against(plan, {"r0": [2, 3, 4, 5]})


def test_host_fallback_keeps_one_step_accounting():
    fallback_result().validate_against(base_plan(), {"r0": [3]})
    with pytest.raises(ValueError, match="one-step vLLM semantics"):
        replace(fallback_result(), computed_steps={"r0": 2}, model_calls=2).validate_against(base_plan(), {"r0": [3, 4]})


@pytest.mark.parametrize("state", [EpochCommitState.PREPARED, EpochCommitState.EXECUTING])
def test_device_result_requires_committed_state(state):
    plan = base_plan()
    with pytest.raises(ValueError, match="not committed"):
        device_result(plan, {"r0": 4}, commit_state=state).validate_against(plan, {"r0": [2, 3, 4, 5]})


def test_host_fallback_rejects_device_owned_request():
    plan = base_plan(base_request(state_owner="device"))
    with pytest.raises(ValueError, match="Host no longer owns"):
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
    with pytest.raises(ValueError, match="did not commit"):
        plain.validate_against(plan, tokens)
    proven = replace(plain, kv_imported=True, kv_import_checksum=123, kv_snapshot_checksum=123)
    proven.validate_against(plan, tokens)
    with pytest.raises(ValueError, match="equivalent imported KV"):
        replace(proven, kv_import_checksum=124).validate_against(plan, tokens)
    # a device-IPC import needs only a non-zero import checksum
    replace(plain, kv_imported=True, kv_import_checksum=5, kv_transfer_mode="device_ipc").validate_against(plan, tokens)
    with pytest.raises(ValueError, match="did not prove an imported KV transfer"):
        replace(plain, kv_imported=True, kv_import_checksum=0, kv_transfer_mode="device_ipc").validate_against(plan, tokens)
    with pytest.raises(ValueError, match="mode is set without an import"):
        replace(plain, kv_transfer_mode="device_ipc").validate_against(base_plan(), tokens)
    with pytest.raises(ValueError, match="Host-owned"):
        base_plan(base_request(kv_import_required=True, state_owner="device")).validate()


@pytest.mark.parametrize(
    ("result_kw", "message"),
    [
        ({"status": 3}, "failed device execution"),
        ({"feed_calls": 2}, "exactly one Feed and one Fetch"),
        ({"row_generations": (5,)}, "generations disagree"),
        ({"model_calls": 3}, "model-call count"),
        ({"version": CONTRACT_VERSION + 1}, "version mismatch"),
        ({"computed_steps": {"r0": 9}}, "outside the epoch"),
        ({"computed_steps": {"x": 4}}, "request set mismatch"),
    ],
)
def test_device_result_rules(result_kw, message):
    plan = base_plan()
    result = replace(device_result(plan, {"r0": 4}), **result_kw)
    with pytest.raises(ValueError, match=message):
        result.validate_against(plan, {"r0": [2, 3, 4, 5]})


def test_sampled_tokens_must_match_steps():
    plan = base_plan()
    with pytest.raises(ValueError, match="sampled token count"):
        device_result(plan, {"r0": 4}).validate_against(plan, {"r0": [2, 3]})
    with pytest.raises(ValueError, match="output request set mismatch"):
        device_result(plan, {"r0": 4}).validate_against(plan, {})


@pytest.mark.parametrize(
    ("plan_fn", "message"),
    [
        (lambda: replace(base_plan(), version=2), "unsupported resident epoch contract"),
        (lambda: base_plan(batch=3), "graph batch size"),
        (lambda: replace(base_plan(), active_mask=(1, 0)), "active mask does not match graph batch size"),
        (lambda: replace(base_plan(batch=2), active_mask=(1, 2)), "only zero or one"),
        (lambda: ResidentEpochPlan(CONTRACT_VERSION, 2, 4, 8, (base_request(), base_request(row=1, generation=2)),
                                   (1, 1)),
         "request IDs must be unique"),
        (lambda: ResidentEpochPlan(CONTRACT_VERSION, 2, 4, 8,
                                   (base_request(), base_request(req_id="r1", generation=2)), (1, 1)),
         "resident rows must be unique"),
        (lambda: base_plan(base_request(generation=0)), "generations must be positive"),
        (lambda: ResidentEpochPlan(CONTRACT_VERSION, 2, 4, 8,
                                   (base_request(), base_request(req_id="r1", row=1)), (1, 1)),
         "generations must be unique"),
        (lambda: ResidentEpochPlan(CONTRACT_VERSION, 1, 4, 8, (base_request(row=1),), (1,)), "outside the static graph"),
        (lambda: base_plan(base_request(sequence_length=3)), "sequence length and position disagree"),
        (lambda: base_plan(base_request(state_owner="gpu")), "invalid state owner"),
        (lambda: base_plan(base_request(position=5, sequence_length=6)), "exceeds logical capacity"),
        (lambda: replace(base_plan(base_request(), batch=2), active_mask=(0, 1)), "does not match resident rows"),
        (lambda: ResidentEpochPlan(CONTRACT_VERSION, 1, 4, 8, (), (0,)), "does not fit the static graph"),
    ],
)
def test_plan_validation_rules(plan_fn, message):
    with pytest.raises(ValueError, match=message):
        plan_fn().validate()


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
