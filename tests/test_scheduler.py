"""Scheduler-side K selection, rows and generations (cruise_amd.scheduler)
over an in-memory vLLM-shaped base scheduler (tests/fake_vllm.py).

Restates the scenarios of the reference's tests/test_real_scheduler.py
(fixed-graph plans for 1-4 requests, host prefill handing rows to device
ownership with a KV import, continuous admission with host isolation and row
reuse, ineligible requests kept on the host lane) and
tests/test_scheduler_accounting.py (computed tokens advance by the steps the
device ran), plus the K-selection rule, the row/generation allocator,
eligibility reasons, configuration and benchmark counters.
"""
from __future__ import annotations

import json
import os
import uuid
from pathlib import Path
from types import SimpleNamespace

import pytest

from cruise_amd.backend import ModelRunnerOutput
from cruise_amd.config import ResidentEpochConfig
from cruise_amd.contract import (
    CONTRACT_VERSION,
    EpochCommitState,
    ResidentEpochPlan,
    ResidentEpochRequest,
    ResidentEpochResult,
    attach_plan,
    attach_result,
    get_plan,
)
from cruise_amd.eligibility import request_rejection_reason
from cruise_amd.scheduler import ResidentEpochSchedulerMixin, ResidentRowTable, epoch_steps_for, host_lane_reason
from fake_vllm import EOS_TOKEN_ID, FakeScheduler, Request, RequestStatus, greedy_params, qwen7b_vllm_config


class Scheduler(ResidentEpochSchedulerMixin, FakeScheduler):
    pass


def make_scheduler(batch_size: int, max_steps: int = 8) -> Scheduler:
    s = Scheduler(max_num_seqs=batch_size)
    s._resident_epoch_config = ResidentEpochConfig(max_steps=max_steps)
    return s


def greedy_requests(s: Scheduler, count: int, max_tokens: int = 8) -> list[Request]:
    reqs = [Request(str(i), [i + 1], greedy_params(max_tokens)) for i in range(count)]
    for r in reqs:
        s.add_request(r)
    return reqs


def prefill_request(rid: str, prompt: list[int], max_tokens: int) -> Request:
    return Request(rid, list(prompt), greedy_params(max_tokens))


def host_step(s, output, tokens_by_req):
    ids = list(output.num_scheduled_tokens)
    s.update_from_output(output, ModelRunnerOutput(ids, {r: i for i, r in enumerate(ids)},
                                                    [tokens_by_req[r] for r in ids]))


def commit_device_epoch(s, output, tokens_by_req):
    plan = get_plan(output)
    assert plan is not None
    ids = list(plan.req_ids)
    mro = ModelRunnerOutput(ids, {r: i for i, r in enumerate(ids)}, [tokens_by_req[r] for r in ids])
    importing = any(r.kv_import_required for r in plan.requests)
    attach_result(mro, ResidentEpochResult(
        version=CONTRACT_VERSION, route="device", status=0, model_calls=max(len(t) for t in tokens_by_req.values()),
        computed_steps={r: len(tokens_by_req[r]) for r in ids}, row_generations=plan.row_generations,
        kv_imported=importing, kv_import_checksum=1 if importing else 0, kv_snapshot_checksum=1 if importing else 0,
    ))
    s.update_from_output(output, mro)


# ---------------------------------------------------------------------------
# K selection and allocation rules
# ---------------------------------------------------------------------------
@pytest.mark.parametrize(
    ("max_steps", "remaining", "k"),
    [(8, [8], 8), (8, [7], 4), (8, [3, 9], 2), (4, [100], 4), (2, [6, 1], 1), (8, [5, 6, 7], 4), (1, [8], 1)],
)
def test_epoch_length_is_largest_power_within_budget(max_steps, remaining, k):
    assert epoch_steps_for(max_steps, remaining) == k


def rows_of(table):
    return {rid: seat.row for rid, seat in table.seats.items()}


def generations_of(table):
    return {rid: seat.generation for rid, seat in table.seats.items()}


def test_rows_are_lowest_free_and_generations_fresh():
    t = ResidentRowTable(4)
    t.seat_exactly(("a", "b", "c"))
    assert rows_of(t) == {"a": 0, "b": 1, "c": 2}
    assert generations_of(t) == {"a": 1, "b": 2, "c": 3}
    t.device_owned.add("b")
    t.seat_exactly(("a", "c", "d", "e"))  # b leaves: its row is reused first
    assert rows_of(t) == {"a": 0, "c": 2, "d": 1, "e": 3}
    assert generations_of(t)["d"] == 4 and generations_of(t)["e"] == 5
    assert "b" not in t.device_owned
    with pytest.raises(RuntimeError, match="exhausted"):
        t.seat_exactly(("a", "c", "d", "e", "f"))


def test_generation_space_is_bounded():
    t = ResidentRowTable(4, first_generation=2**31 - 1)
    assert t.admit("last").generation == 2**31 - 1
    with pytest.raises(RuntimeError, match="generation space exhausted"):
        t.admit("x")


def test_scheduler_without_init_gets_default_state():
    s = Scheduler.__new__(Scheduler)
    config, table = s._resident_state()
    assert config == ResidentEpochConfig() and table.rows == 4 and s._resident_epoch_device_owned == set()


# ---------------------------------------------------------------------------
# Scenarios of the reference's scheduler tests
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("batch_size", [1, 2, 3, 4])
def test_fixed_graph_plan_and_committed_epoch(batch_size):
    s = make_scheduler(batch_size)
    reqs = greedy_requests(s, batch_size)
    out = s.schedule()
    plan = get_plan(out)
    assert plan is not None and plan.graph_batch_size == 4 and plan.max_steps == 8
    assert plan.active_mask == (1,) * batch_size + (0,) * (4 - batch_size)
    assert all(n == 1 for n in out.num_scheduled_tokens.values())
    assert all(len(r.scheduler_block_ids) == 1 for r in plan.requests)
    assert [r.row for r in plan.requests] == list(range(batch_size))
    assert [r.generation for r in plan.requests] == list(range(1, batch_size + 1))
    assert all(r.position == 0 and r.sequence_length == 1 and r.token_id == int(r.req_id) + 1 for r in plan.requests)
    commit_device_epoch(s, out, {r: [100 + k for k in range(8)] for r in plan.req_ids})
    for r in reqs:
        assert (r.num_computed_tokens, r.num_tokens, r.num_output_tokens) == (8, 9, 8)
        assert r.status == RequestStatus.FINISHED_LENGTH_CAPPED


def test_unsupported_sampling_stays_on_host_path():
    s = make_scheduler(1)
    reqs = greedy_requests(s, 1)
    reqs[0].sampling_params.temperature = 0.8
    out = s.schedule()
    assert get_plan(out) is None
    assert s._resident_epoch_last_rejection == "non-greedy-temperature"
    assert s.num_lookahead_tokens == 0
    assert s.kv_cache_manager.get_blocks("0").get_block_ids() == ([0],)


def test_short_epoch_at_eos_finishes_the_request():
    s = make_scheduler(2)
    reqs = greedy_requests(s, 2, max_tokens=8)
    out = s.schedule()
    commit_device_epoch(s, out, {"0": [5, 6, EOS_TOKEN_ID], "1": list(range(10, 18))})
    assert reqs[0].status == RequestStatus.FINISHED_STOPPED and reqs[0].num_computed_tokens == 3
    assert reqs[1].status == RequestStatus.FINISHED_LENGTH_CAPPED


def test_host_prefill_transitions_to_device_owned_decode():
    s = make_scheduler(1)
    req = Request("p", [7, 8, 9], greedy_params(4))
    s.add_request(req)
    prefill = s.schedule()
    assert get_plan(prefill) is None and s._resident_epoch_last_rejection == "not-single-token-decode"
    host_step(s, prefill, {"p": [101]})
    assert (req.num_computed_tokens, req.num_output_tokens) == (3, 1)
    first = s.schedule()
    plan = get_plan(first)
    assert plan is not None and plan.max_steps == 2
    r0 = plan.requests[0]
    assert (r0.position, r0.sequence_length, r0.token_id, r0.state_owner, r0.kv_import_required) == (3, 4, 101, "host", True)
    commit_device_epoch(s, first, {"p": [102, 103]})
    assert "p" in s._resident_epoch_device_owned
    nxt = get_plan(s.schedule())
    assert nxt is not None and nxt.requests[0].state_owner == "device" and not nxt.requests[0].kv_import_required


def test_continuous_admission_isolates_host_prefill_and_reuses_rows():
    s = make_scheduler(2, max_steps=2)
    a = prefill_request("A", [9707, 11], 7)
    s.add_request(a)
    prefill_a = s.schedule()
    assert get_plan(prefill_a) is None
    host_step(s, prefill_a, {"A": [101]})
    import_a = s.schedule()
    assert get_plan(import_a).max_steps == 2
    commit_device_epoch(s, import_a, {"A": [102, 103]})

    b = prefill_request("B", [9707, 11, 358], 2)
    s.add_request(b)
    prefill_b = s.schedule()
    assert get_plan(prefill_b) is None and prefill_b.num_scheduled_tokens == {"B": 3}
    assert s._resident_epoch_last_rejection == "host-prefill-admission"
    assert [r.request_id for r in s.running] == ["A", "B"]
    host_step(s, prefill_b, {"B": [201]})
    import_b = s.schedule()
    plan_b = get_plan(import_b)
    assert plan_b.max_steps == 1
    assert [(r.req_id, r.row, r.generation) for r in plan_b.requests] == [("A", 0, 1), ("B", 1, 2)]
    assert [(r.state_owner, r.kv_import_required) for r in plan_b.requests] == [("device", False), ("host", True)]
    commit_device_epoch(s, import_b, {"A": [104], "B": [202]})
    assert b.status == RequestStatus.FINISHED_LENGTH_CAPPED

    c = prefill_request("C", [9707, 11, 358, 374], 2)
    s.add_request(c)
    prefill_c = s.schedule()
    assert get_plan(prefill_c) is None and prefill_c.num_scheduled_tokens == {"C": 4}
    assert s._resident_epoch_last_rejection == "host-prefill-admission"
    host_step(s, prefill_c, {"C": [301]})
    import_c = s.schedule()
    plan_c = get_plan(import_c)
    assert [(r.req_id, r.row, r.generation) for r in plan_c.requests] == [("A", 0, 1), ("C", 1, 3)]
    assert plan_c.requests[1].kv_import_required
    commit_device_epoch(s, import_c, {"A": [105], "C": [302]})
    assert c.status == RequestStatus.FINISHED_LENGTH_CAPPED

    finish = s.schedule()
    plan_f = get_plan(finish)
    assert plan_f.req_ids == ("A",) and plan_f.max_steps == 2
    commit_device_epoch(s, finish, {"A": [106, 107]})
    assert a.status == RequestStatus.FINISHED_LENGTH_CAPPED


def test_ineligible_admission_uses_host_lane_without_advancing_device_request():
    s = make_scheduler(2, max_steps=2)
    a = prefill_request("A", [9707, 11], 7)
    s.add_request(a)
    p = s.schedule()
    host_step(s, p, {"A": [101]})
    commit_device_epoch(s, s.schedule(), {"A": [102, 103]})
    computed_a = a.num_computed_tokens

    u = prefill_request("u", [9707, 11], 2)
    u.sampling_params.temperature = 0.8
    s.add_request(u)
    up = s.schedule()
    assert get_plan(up) is None and up.num_scheduled_tokens == {"u": 2}
    assert s._resident_epoch_last_rejection == "host-prefill-admission"
    host_step(s, up, {"u": [201]})
    ud = s.schedule()
    assert get_plan(ud) is None and ud.num_scheduled_tokens == {"u": 1}
    assert s._resident_epoch_last_rejection == "unsupported-host-isolation"
    host_step(s, ud, {"u": [202]})
    assert u.status == RequestStatus.FINISHED_LENGTH_CAPPED
    assert a.num_computed_tokens == computed_a  # the device-owned request never ran on the host
    resume = get_plan(s.schedule())
    assert resume.req_ids == ("A",) and resume.requests[0].state_owner == "device"
    assert resume.requests[0].generation == 1


def test_two_simultaneous_prefills_are_isolated_from_device_owned_request():
    s = make_scheduler(3, max_steps=2)
    a = prefill_request("A", [9707, 11], 7)
    s.add_request(a)
    p = s.schedule()
    host_step(s, p, {"A": [101]})
    commit_device_epoch(s, s.schedule(), {"A": [102, 103]})
    s.add_request(prefill_request("B", [9707, 11, 358], 3))
    s.add_request(prefill_request("C", [9707, 11, 358, 374], 3))
    bc = s.schedule()
    assert get_plan(bc) is None and bc.num_scheduled_tokens == {"B": 3, "C": 4}
    assert s._resident_epoch_last_rejection == "host-prefill-admission"
    host_step(s, bc, {"B": [201], "C": [301]})
    plan = get_plan(s.schedule())
    assert plan.req_ids == ("A", "B", "C")
    assert [r.state_owner for r in plan.requests] == ["device", "host", "host"]
    assert [r.kv_import_required for r in plan.requests] == [False, True, True]


def test_running_prefill_is_isolated_from_device_owned_requests():
    s = make_scheduler(2)
    device_req = greedy_requests(s, 1, max_tokens=6)[0]
    prefill = prefill_request("prefill", [9707, 11, 358], 4)
    prefill.num_computed_tokens = 1
    s.running = [device_req, prefill]
    assert host_lane_reason(s, [device_req]) == "host-prefill-admission"
    assert host_lane_reason(s, []) is None


def test_device_owned_request_is_never_sent_to_the_host():
    # a block-size mismatch makes the plan impossible while the request is device-owned
    s2 = make_scheduler(1)
    r = greedy_requests(s2, 1, max_tokens=20)[0]
    out = s2.schedule()
    commit_device_epoch(s2, out, {"0": list(range(1, 9))})
    s2.block_size = 64
    with pytest.raises(RuntimeError, match="device-owned requests cannot run on the host: 0"):
        s2.schedule()
    assert r.request_id in s2._resident_epoch_device_owned


@pytest.mark.parametrize(
    ("mutate", "reason"),
    [
        (lambda s, r: setattr(s, "block_size", 16), "block-size"),
        (lambda s, r: setattr(s, "connector", object()), "cache-connector"),
        (lambda s, r: setattr(r[0], "prompt_token_ids", list(range(1, 10))), "not-single-token-decode"),
    ],
)
def test_batch_level_rejections(mutate, reason):
    s = make_scheduler(1)
    reqs = greedy_requests(s, 1)
    mutate(s, reqs)
    assert get_plan(s.schedule()) is None
    assert s._resident_epoch_last_rejection == reason


def test_empty_schedule_is_rejected():
    s = make_scheduler(1)
    assert get_plan(s.schedule()) is None and s._resident_epoch_last_rejection == "empty-schedule"


def test_epoch_that_would_pass_capacity_is_rejected():
    s = make_scheduler(1)
    s._resident_epoch_config = ResidentEpochConfig(max_steps=8, logical_capacity=8)
    r = Request("p", [1, 2, 3, 4, 5, 6], greedy_params(8))  # position 6, K = 4: 6 + 4 > 8
    s.add_request(r)
    host_step(s, s.schedule(), {"p": [7]})
    assert get_plan(s.schedule()) is None
    assert s._resident_epoch_last_rejection == "logical-capacity"


# ---------------------------------------------------------------------------
# Accounting (test_scheduler_accounting.py:52-116)
# ---------------------------------------------------------------------------
def accounting_case(route):
    s = Scheduler.__new__(Scheduler)
    s.requests = {"r0": SimpleNamespace(num_computed_tokens=1, num_tokens=1)}
    out = SimpleNamespace(num_scheduled_tokens={"r0": 1})
    plan = ResidentEpochPlan(CONTRACT_VERSION, 1, 4, 8, (ResidentEpochRequest("r0", 0, 1, 1, 0, 1, 9, (4,), (0, 1)),),
                             (1,))
    attach_plan(out, plan)
    if route == "device":
        mro = ModelRunnerOutput(["r0"], {"r0": 0}, [[2, 3, 4, 5]])
        result = ResidentEpochResult(CONTRACT_VERSION, "device", 0, 4, {"r0": 4}, row_generations=(1,))
    else:
        mro = ModelRunnerOutput(["r0"], {"r0": 0}, [[2]])
        result = ResidentEpochResult(CONTRACT_VERSION, "host_fallback", 0, 1, {"r0": 1},
                                     commit_state=EpochCommitState.PREPARED, fallback_safe=True, feed_calls=0,
                                     fetch_calls=0)
    attach_result(mro, result)
    s._apply_resident_epoch_accounting(out, mro, plan, result)
    return s.requests["r0"].num_computed_tokens


def test_device_epoch_advances_computed_tokens_by_actual_steps():
    assert accounting_case("device") == 4


def test_host_fallback_retains_normal_one_step_accounting():
    assert accounting_case("host_fallback") == 1


# ---------------------------------------------------------------------------
# Construction, eligibility, configuration, counters
# ---------------------------------------------------------------------------
def test_constructor_rejects_unsupported_deployments(monkeypatch):
    monkeypatch.delenv("VLLM_ASCEND_RESIDENT_EPOCH_STEPS", raising=False)
    Scheduler(vllm_config=qwen7b_vllm_config())
    with pytest.raises(ValueError, match="hidden_size=3584.*has 4096"):
        Scheduler(vllm_config=qwen7b_vllm_config(hidden_size=4096))
    with pytest.raises(ValueError, match="need synchronous scheduling"):
        Scheduler(async_scheduling=True)
    cfg = qwen7b_vllm_config()
    cfg.parallel_config.tensor_parallel_size = 2
    with pytest.raises(ValueError, match="tensor and pipeline parallel size"):
        Scheduler(vllm_config=cfg)
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_STEPS", "3")
    with pytest.raises(ValueError, match=r"max_steps=3 is not one of \(1, 2, 4, 8\)"):
        Scheduler()


def eligible_request(**overrides):
    params = greedy_params(8)
    req = SimpleNamespace(pooling_params=None, mm_features=[], lora_request=None, prompt_embeds=None,
                          use_structured_output=False, sampling_params=params)
    for k, v in overrides.items():
        setattr(params if hasattr(params, k) else req, k, v)
    return req


@pytest.mark.parametrize(
    ("field", "value", "reason"),
    [
        ("temperature", 0.8, "non-greedy-temperature"),
        ("top_k", 8, "unsupported-sampling-filter"),
        ("presence_penalty", 0.1, "sampling-penalty"),
        ("min_tokens", 2, "min-tokens"),
        ("ignore_eos", True, "ignore-eos"),
        ("stop_token_ids", [7], "extra-stop-condition"),
        ("logprobs", 1, "logprobs"),
        ("allowed_token_ids", [1, 2], "logit-processor"),
        ("bad_words", ["x"], "bad-words"),
        ("eos_token_id", None, "missing-eos"),
        ("pooling_params", object(), "pooling-request"),
        ("lora_request", object(), "lora"),
        ("use_structured_output", True, "structured-output"),
        ("sampling_params", None, "missing-sampling-params"),
    ],
)
def test_unsupported_semantics_are_rejected(field, value, reason):
    assert request_rejection_reason(eligible_request()) is None
    assert request_rejection_reason(eligible_request(**{field: value})) == reason


def test_config_geometry_and_mapping():
    c = ResidentEpochConfig(logical_capacity=256)
    assert [c.row_blocks(r) for r in range(4)] == [(0, 1), (2, 3), (4, 5), (6, 7)]
    assert [c.epoch_steps(b) for b in (1, 2, 3, 5, 8, 100)] == [1, 2, 2, 4, 8, 8]
    with pytest.raises(ValueError):
        c.epoch_steps(0)
    assert ResidentEpochConfig.from_env({"VLLM_ASCEND_RESIDENT_EPOCH_STEPS": "2"}).max_steps == 2
    assert len(ResidentEpochConfig(max_steps=3, logical_capacity=1, max_batch_size=2).problems()) == 3


def test_config_from_env(monkeypatch):
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_STEPS", "4")
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_CAPACITY", "256")
    assert ResidentEpochConfig.from_env() == ResidentEpochConfig(max_steps=4, logical_capacity=256)
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_CAPACITY", "2")
    with pytest.raises(ValueError, match="cannot hold an epoch of 4 steps"):
        ResidentEpochConfig.from_env()
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_CAPACITY", "x")
    with pytest.raises(ValueError, match="is not an integer"):
        ResidentEpochConfig.from_env()
