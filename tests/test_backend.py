"""Worker backend (cruise_amd.backend) with engine doubles, on the CPU:
every failure surfaces as a ResidentEpochExecutionError with the commit state
the reference assigns to it (backend.py:68-208)."""
from __future__ import annotations

import pytest

from cruise_amd.backend import NativeEpochOutput, NativeWarmupOutput, ResidentEpochBackend, load_backend_from_env
from cruise_amd.contract import (
    CONTRACT_VERSION,
    EpochCommitState,
    ResidentEpochExecutionError,
    ResidentEpochPlan,
    ResidentEpochRequest,
    get_result,
)
from cruise_amd.kv_transfer import IPC_KEY_BYTES, DeviceKVTransfer, KVGeometry, ResidentKVSnapshot, kv_payload_checksum

G = KVGeometry(layers=2, batch=4, block_size=4, kv_heads=1, head_size=8, element_bytes=2)


def req(row, gen, tok=5, pos=0, imp=False):
    return ResidentEpochRequest(f"r{row}", row, gen, tok, pos, pos + 1, 9, (row,), (2 * row, 2 * row + 1),
                                kv_import_required=imp)


def plan(*reqs, steps=4):
    mask = [0] * 4
    for r in reqs:
        mask[r.row] = 1
    return ResidentEpochPlan(CONTRACT_VERSION, 4, steps, 8, tuple(reqs), tuple(mask))


class Engine:
    """Runs every row to the plan's K emitting 10 * row + step."""

    def __init__(self, **override):
        self.override = override
        self.calls = []

    def _out(self, p, **kw):
        tokens = {r.req_id: [10 * r.row + s for s in range(p.max_steps)] for r in p.requests}
        fields = dict(status=0, model_calls=p.max_steps, token_ids=tokens, row_generations=p.row_generations)
        fields.update(kw)
        fields.update(self.override)
        return NativeEpochOutput(**fields)

    def warm_up(self):
        return NativeWarmupOutput(status=0, model_calls=1, feed_calls=1, fetch_calls=1, wall_us=3)

    def execute(self, p):
        self.calls.append("execute")
        return self._out(p)

    def execute_with_import(self, p, snap):
        self.calls.append("import")
        return self._out(p, kv_imported=True, kv_import_checksum=snap.checksum)

    def execute_with_device_transfer(self, p, t):
        self.calls.append("ipc")
        return self._out(p, kv_imported=True, kv_import_checksum=77)


def snapshot(mask, gens):
    payload = bytes(range(256)) * (G.payload_bytes // 256)
    return ResidentKVSnapshot(3, mask, gens, payload, kv_payload_checksum(payload, mask, G), G)


def transfer(mask, gens, blocks):
    return DeviceKVTransfer(4, mask, gens, blocks, 64 * G.block_bytes, (0,) * 4, (b"\x07" * IPC_KEY_BYTES,) * 4, G)


def test_device_epoch_becomes_model_runner_output():
    out = ResidentEpochBackend(Engine()).execute(plan(req(1, 3), req(3, 4)))
    assert out.req_ids == ["r1", "r3"] and out.req_id_to_index == {"r1": 0, "r3": 1}
    assert out.sampled_token_ids == [[10, 11, 12, 13], [30, 31, 32, 33]]
    result = get_result(out)
    assert result.route == "device" and result.commit_state == EpochCommitState.COMMITTED
    assert result.computed_steps == {"r1": 4, "r3": 4} and result.kv_transfer_mode == "none"


def test_import_modes_are_proven():
    p = plan(req(1, 3, imp=True), req(3, 4))
    eng = Engine()
    out = ResidentEpochBackend(eng).execute(p, snapshot=snapshot(0b0010, (0, 3, 0, 0)))
    r = get_result(out)
    assert r.kv_transfer_mode == "host_snapshot" and r.kv_snapshot_checksum == r.kv_import_checksum != 0
    out = ResidentEpochBackend(eng).execute(p, device_transfer=transfer(0b0010, (0, 3, 0, 0), (0, 1, 0, 0)))
    assert get_result(out).kv_transfer_mode == "device_ipc"
    assert eng.calls == ["import", "ipc"]
    with pytest.raises(ValueError, match="one source"):
        ResidentEpochBackend(eng).execute(p, snapshot=snapshot(0b0010, (0, 3, 0, 0)),
                                          device_transfer=transfer(0b0010, (0, 3, 0, 0), (0, 1, 0, 0)))


@pytest.mark.parametrize(
    ("override", "state", "message"),
    [
        ({"status": 207}, EpochCommitState.COMMITTED, "fell back with status 207"),
        ({"commit_state": EpochCommitState.EXECUTING}, EpochCommitState.EXECUTING, "did not commit"),
        ({"token_ids": {"rX": [1]}}, EpochCommitState.COMMITTED, "answered for"),
        ({"model_calls": 9}, EpochCommitState.COMMITTED, "output is invalid"),
        ({"feed_calls": 2}, EpochCommitState.COMMITTED, "device-round-trip"),
    ],
)
def test_failures_carry_their_commit_state(override, state, message):
    with pytest.raises(ResidentEpochExecutionError, match=message) as err:
        ResidentEpochBackend(Engine(**override)).execute(plan(req(0, 1)))
    assert err.value.commit_state == state


def test_snapshot_checksum_disagreement_is_committed_failure():
    p = plan(req(1, 3, imp=True))
    with pytest.raises(ResidentEpochExecutionError, match="disagrees with the host") as err:
        ResidentEpochBackend(Engine(kv_import_checksum=5)).execute(p, snapshot=snapshot(0b0010, (0, 3, 0, 0)))
    assert err.value.commit_state == EpochCommitState.COMMITTED
    with pytest.raises(ResidentEpochExecutionError, match="returned no checksum"):
        ResidentEpochBackend(Engine(kv_import_checksum=0)).execute(
            p, device_transfer=transfer(0b0010, (0, 3, 0, 0), (0, 1, 0, 0)))


def test_invalid_plan_is_prepared_failure():
    bad = ResidentEpochPlan(CONTRACT_VERSION, 4, 4, 8, (req(0, 1),), (1, 1, 0, 0))
    eng = Engine()
    with pytest.raises(ResidentEpochExecutionError, match="rejected before execution") as err:
        ResidentEpochBackend(eng).execute(bad)
    assert err.value.input_preserving and eng.calls == []


def test_engine_exception_is_executing_failure():
    class Broken(Engine):
        def execute(self, p):
            raise OSError("socket reset")

    with pytest.raises(ResidentEpochExecutionError, match="without proof of its commit state") as err:
        ResidentEpochBackend(Broken()).execute(plan(req(0, 1)))
    assert err.value.commit_state == EpochCommitState.EXECUTING


def test_engine_errors_with_a_commit_state_pass_through():
    class Declared(Engine):
        def execute(self, p):
            raise ResidentEpochExecutionError("socket closed before send", commit_state=EpochCommitState.PREPARED,
                                              status=13)

    with pytest.raises(ResidentEpochExecutionError, match="socket closed before send") as err:
        ResidentEpochBackend(Declared()).execute(plan(req(0, 1)))
    assert err.value.input_preserving and err.value.status == 13


def test_missing_import_support_is_prepared_failure():
    class Plain:
        def execute(self, p):
            raise AssertionError

    with pytest.raises(ResidentEpochExecutionError, match="no execute_with_import") as err:
        ResidentEpochBackend(Plain()).execute(plan(req(1, 3, imp=True)), snapshot=snapshot(0b0010, (0, 3, 0, 0)))
    assert err.value.input_preserving


def test_warm_up_requires_one_complete_step():
    ResidentEpochBackend(Engine()).warm_up()

    class Partial(Engine):
        def warm_up(self):
            return NativeWarmupOutput(status=0, model_calls=0, feed_calls=1, fetch_calls=1, wall_us=0)

    with pytest.raises(RuntimeError, match="one complete decoder step"):
        ResidentEpochBackend(Partial()).warm_up()


def test_backend_factory_from_env(monkeypatch):
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY", f"{__name__}:Engine")
    assert isinstance(load_backend_from_env().engine, Engine)
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_BACKEND_FACTORY", "nocolon")
    with pytest.raises(RuntimeError, match="module:factory"):
        load_backend_from_env()
