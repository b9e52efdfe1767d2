"""Sidecar protocol and server, on the CPU.

The wire-record tests restate the reference's tests/test_sidecar_protocol.py
(record sizes and field order, the warm-up request, a device-IPC request
reported as a KV import).  The server tests build resident_epoch_server
from its source against a test double of the engine's C-ABI
(tests/native/stub_engine.cpp) and drive every operation of the protocol
through the Python client, as the reference's worker does
(sidecar_backend.py:67-462; native/resident_epoch_server.cpp:133-216).
"""
from __future__ import annotations

import os
import socket
import subprocess
import uuid
from pathlib import Path

import pytest

from cruise_amd.backend import ResidentEpochBackend
from cruise_amd.build import build_server
from cruise_amd.contract import (
    CONTRACT_VERSION,
    EpochCommitState,
    ResidentEpochExecutionError,
    ResidentEpochPlan,
    ResidentEpochRequest,
    get_result,
)
from cruise_amd.kv_transfer import (
    IPC_KEY_BYTES,
    IPC_METADATA_BYTES,
    DeviceKVTransfer,
    KVGeometry,
    ResidentKVSnapshot,
    kv_payload_checksum,
)
from cruise_amd.ctypes_backend import CtypesDataFlowEngine
from cruise_amd.sidecar_backend import (
    DEVICE_IPC_EXECUTE,
    EXECUTE,
    GRAPH_BATCH_SIZE,
    PROTOCOL_VERSION,
    REQUEST,
    REQUEST_MAGIC,
    RESPONSE,
    RESPONSE_MAGIC,
    WARM_UP,
    WARMUP_GENERATION,
    SidecarDataFlowEngine,
    decode_response,
)

ROOT = Path(__file__).resolve().parents[1]


def request(row, gen, token, pos, *, req_id=None, imp=False, block=0):
    return ResidentEpochRequest(
        req_id=req_id or f"r{row}", row=row, generation=gen, token_id=token, position=pos,
        sequence_length=pos + 1, eos_token_id=151645, scheduler_block_ids=(block,),
        device_block_ids=(2 * row, 2 * row + 1), kv_import_required=imp,
    )


def plan_of(*reqs, steps=4, capacity=8):
    mask = [0] * 4
    for r in reqs:
        mask[r.row] = 1
    return ResidentEpochPlan(CONTRACT_VERSION, 4, steps, capacity, tuple(reqs), tuple(mask))


# ---------------------------------------------------------------------------
# Wire records (test_sidecar_protocol.py:23-161)
# ---------------------------------------------------------------------------
def test_record_sizes_and_field_order():
    assert (REQUEST.size, RESPONSE.size) == (136, 352)
    raw = REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, EXECUTE, 2, 4, 0, *range(4), *range(4), *([1] * 4),
                       *([151645] * 4), 1, 2, 0, 0)
    assert REQUEST.unpack(raw)[:5] == (REQUEST_MAGIC, PROTOCOL_VERSION, EXECUTE, 2, 4)
    resp = RESPONSE.pack(RESPONSE_MAGIC, 0, 0, 4, 1, 1, EpochCommitState.COMMITTED, 0x12345678, 123, 45, 260, 368,
                         4, 4, 0, 0, 1, 2, 0, 0, *range(32))
    v = RESPONSE.unpack(resp)
    assert v[:6] == (RESPONSE_MAGIC, 0, 0, 4, 1, 1)
    assert v[6:12] == (EpochCommitState.COMMITTED, 0x12345678, 123, 45, 260, 368)
    assert v[20:] == tuple(range(32))


class FakeLink:
    """Stands in for the socket: records what is sent and answers with one
    fixed response record."""

    def __init__(self, *response):
        self.sent = []
        self.response = RESPONSE.pack(*response)

    def exchange(self, record):
        self.sent.append(record)
        return decode_response(self.response)

    def close(self):
        pass


def engine_with(link):
    eng = SidecarDataFlowEngine.__new__(SidecarDataFlowEngine)
    eng.link = link
    return eng


def test_warmup_request_uses_the_reserved_generation():
    link = FakeLink(RESPONSE_MAGIC, 0, 0, 1, 1, 1, 2, 0, 7, 3, 260, 368, 1, 0, 0, 0,
                    WARMUP_GENERATION, 0, 0, 0, 12, *([-1] * 31))
    out = engine_with(link).warm_up()
    fields = REQUEST.unpack(link.sent[0])
    assert fields[:5] == (REQUEST_MAGIC, PROTOCOL_VERSION, WARM_UP, 1, 1)
    assert fields[6:10] == (11690, 0, 0, 0)
    assert fields[-GRAPH_BATCH_SIZE:] == (WARMUP_GENERATION, 0, 0, 0)
    assert (out.status, out.model_calls, out.feed_calls, out.fetch_calls) == (0, 1, 1, 1)


def test_warmup_must_run_exactly_row_zero():
    link = FakeLink(RESPONSE_MAGIC, 0, 0, 1, 1, 1, 2, 0, 7, 3, 260, 368, 1, 1, 0, 0,
                    WARMUP_GENERATION, 0, 0, 0, *([-1] * 32))
    with pytest.raises(RuntimeError, match="instead of one step on row 0"):
        engine_with(link).warm_up()


def test_plan_rows_are_laid_out_on_the_graph_rows():
    link = FakeLink(RESPONSE_MAGIC, 0, 0, 4, 1, 1, 2, 0, 0, 0, 260, 368, 0, 4, 0, 4, 0, 3, 0, 4, *([-1] * 32))
    plan = plan_of(request(1, 3, 500, 2), request(3, 4, 600, 0))
    engine_with(link).execute(plan)
    fields = REQUEST.unpack(link.sent[0])
    assert fields[3:5] == (2, 4)  # request count, K
    assert fields[6:10] == (0, 500, 0, 600)  # tokens
    assert fields[10:14] == (0, 2, 0, 0)  # positions
    assert fields[14:18] == (0, 3, 0, 1)  # lengths
    assert fields[18:22] == (151645,) * 4  # EOS: the plan's, default elsewhere
    assert fields[22:26] == (0, 3, 0, 4)  # generations


def test_device_ipc_execute_is_reported_as_kv_import():
    link = FakeLink(RESPONSE_MAGIC, 0, 0, 1, 1, 1, EpochCommitState.COMMITTED, 0x12345678, 123, 45, 3776, 368,
                    1, 0, 0, 0, 7, 0, 0, 0, 42, *([-1] * 31))
    plan = plan_of(request(0, 7, 11, 1, imp=True), steps=1)
    metadata = b"\0" * IPC_METADATA_BYTES
    out = engine_with(link)._run(plan, DEVICE_IPC_EXECUTE, 9, metadata, "device_ipc")
    assert out.kv_imported is True and out.kv_transfer_mode == "device_ipc"
    assert out.kv_import_checksum == 0x12345678
    assert out.token_ids == {"r0": [42]}
    assert len(link.sent) == 1 and link.sent[0][REQUEST.size:] == metadata
    assert REQUEST.unpack(link.sent[0][: REQUEST.size])[2] == DEVICE_IPC_EXECUTE


def test_invalid_commit_state_is_ambiguous():
    link = FakeLink(RESPONSE_MAGIC, 0, 0, 1, 1, 1, 9, 0, 0, 0, 0, 0, *([0] * 8), *([-1] * 32))
    with pytest.raises(ResidentEpochExecutionError) as err:
        engine_with(link).execute(plan_of(request(0, 1, 5, 0)))
    assert err.value.commit_state == EpochCommitState.EXECUTING


def test_executed_count_beyond_the_epoch_is_rejected():
    link = FakeLink(RESPONSE_MAGIC, 0, 0, 4, 1, 1, 2, 0, 0, 0, 0, 0, 9, 0, 0, 0, 1, 0, 0, 0, *([-1] * 32))
    with pytest.raises(ResidentEpochExecutionError, match="9 executed steps") as err:
        engine_with(link).execute(plan_of(request(0, 1, 5, 0)))
    assert err.value.commit_state == EpochCommitState.COMMITTED


def test_a_broken_socket_is_an_executing_failure():
    class Dead:
        def exchange(self, record):
            raise ConnectionResetError("peer reset")

    with pytest.raises(ResidentEpochExecutionError, match="no complete answer") as err:
        engine_with(Dead()).execute(plan_of(request(0, 1, 5, 0)))
    assert err.value.commit_state == EpochCommitState.EXECUTING
    closed = engine_with(None)
    with pytest.raises(ResidentEpochExecutionError) as err:
        closed.execute(plan_of(request(0, 1, 5, 0)))
    assert err.value.input_preserving


def test_transfer_must_match_the_plan():
    link = FakeLink(RESPONSE_MAGIC, *([0] * 19), *([-1] * 32))
    eng = engine_with(link)
    eng.transfer_path = Path("/nonexistent/never-written")
    plan = plan_of(request(1, 5, 7, 2, imp=True), steps=2)
    with pytest.raises(ValueError, match="import mask"):
        eng.execute_with_import(plan, small_snapshot(0b0001, (5, 0, 0, 0)))
    with pytest.raises(ValueError, match="row generations"):
        eng.execute_with_import(plan, small_snapshot(0b0010, (0, 6, 0, 0)))
    assert link.sent == []


# ---------------------------------------------------------------------------
# The server binary against the engine test double
# ---------------------------------------------------------------------------
@pytest.fixture(scope="module")
def stub_server(tmp_path_factory):
    out = tmp_path_factory.mktemp("stub")
    lib = out / "libresident_epoch.so"
    cmd = ["g++", "-O1", "-std=c++17", "-shared", "-fPIC", f"-I{ROOT / 'include'}",
           str(ROOT / "tests" / "native" / "stub_engine.cpp"), "-o", str(lib)]
    subprocess.run(cmd, check=True, capture_output=True)
    return build_server(lib, out / "resident_epoch_server")


@pytest.fixture
def sidecar_env(stub_server, tmp_path, monkeypatch):
    shm = Path("/dev/shm") / f"cruise-sidecar-test-{os.getpid()}-{uuid.uuid4().hex[:8]}"
    shm.mkdir()
    files = {}
    for name, content in (("air", b"air"), ("graph", b"{}"), ("func", b"{}"), ("tiling", bytes(72))):
        files[name] = tmp_path / name
        files[name].write_bytes(content)
    log = tmp_path / "stub.log"
    env = {
        "VLLM_ASCEND_RESIDENT_EPOCH_SERVER": str(stub_server),
        "VLLM_ASCEND_RESIDENT_EPOCH_AIR": str(files["air"]),
        "VLLM_ASCEND_RESIDENT_EPOCH_GRAPH_CONFIG": str(files["graph"]),
        "VLLM_ASCEND_RESIDENT_EPOCH_FUNC_CONFIG": str(files["func"]),
        "VLLM_ASCEND_RESIDENT_EPOCH_TILING": str(files["tiling"]),
        "VLLM_ASCEND_RESIDENT_EPOCH_EXTERNAL_WEIGHTS": str(shm),
        "VLLM_ASCEND_RESIDENT_EPOCH_SOCKET": str(shm / "epoch.sock"),
        "VLLM_ASCEND_RESIDENT_EPOCH_STARTUP_TIMEOUT": "60",
        "STUB_LOG": str(log),
    }
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    yield shm, log
    for p in shm.iterdir():
        p.unlink()
    shm.rmdir()


def small_snapshot(mask, gens, seed=1):
    g = KVGeometry(layers=2, batch=4, block_size=4, kv_heads=1, head_size=8, element_bytes=2)
    payload = bytes((seed * 31 + i * 7) & 0xFF for i in range(g.payload_bytes))
    return ResidentKVSnapshot(77, mask, gens, payload, kv_payload_checksum(payload, mask, g), g)


def test_server_serves_every_operation(sidecar_env):
    shm, log = sidecar_env
    eng = SidecarDataFlowEngine()
    try:
        assert eng.process.poll() is None
        warm = eng.warm_up()
        assert (warm.status, warm.model_calls, warm.feed_calls, warm.fetch_calls) == (0, 1, 1, 1)
        backend = ResidentEpochBackend(eng)
        assert backend.warm_up().commit_state == EpochCommitState.COMMITTED

        # plain epoch: two rows, K=4 (the double emits token + step + 1)
        plan = plan_of(request(0, 1, 100, 0), request(2, 2, 200, 3))
        out = backend.execute(plan)
        assert out.req_ids == ["r0", "r2"]
        assert out.sampled_token_ids == [[101, 102, 103, 104], [201, 202, 203, 204]]
        result = get_result(out)
        assert result.route == "device" and result.computed_steps == {"r0": 4, "r2": 4}
        assert result.row_generations == (1, 0, 2, 0) and result.kv_transfer_mode == "none"

        # host-snapshot import: the server hands SOCKET.kv-transfer to the engine and deletes it after
        snap = small_snapshot(0b0010, (0, 5, 0, 0))
        plan = plan_of(request(1, 5, 7, 2, imp=True), steps=2)
        out = backend.execute(plan, snapshot=snap)
        result = get_result(out)
        assert result.kv_imported and result.kv_transfer_mode == "host_snapshot"
        assert result.kv_import_checksum == snap.checksum == result.kv_snapshot_checksum
        assert not (shm / "epoch.sock.kv-transfer").exists()
        assert f"execute {shm / 'epoch.sock.kv-transfer'} 77" in log.read_text()

        # device IPC import: metadata follows the request on the socket
        keys = tuple(bytes([i + 1]) * IPC_KEY_BYTES for i in range(4))
        g = small_snapshot(1, (1, 0, 0, 0)).geometry
        transfer = DeviceKVTransfer(31, 0b0100, (0, 0, 9, 0), (0, 0, 3, 0), 16 * g.block_bytes,
                                    (0, 0, 4 * g.block_bytes, 4 * g.block_bytes), keys, g)
        plan = plan_of(request(2, 9, 50, 1, imp=True, block=3), steps=1)
        out = backend.execute(plan, device_transfer=transfer)
        result = get_result(out)
        assert result.kv_transfer_mode == "device_ipc"
        assert result.kv_import_checksum == 0x1000 + 0b0100 + 16 * 3
        assert out.sampled_token_ids == [[51]]
    finally:
        eng.close()
    assert eng.process.returncode == 0
    assert not (shm / "epoch.sock").exists()
    lines = log.read_text().splitlines()
    assert lines[0].startswith("create ") and lines[-1] == "destroy"


def test_transport_errors_keep_the_connection(sidecar_env):
    eng = SidecarDataFlowEngine()
    try:
        # request count that disagrees with the rows: the engine's status 12
        link = eng.link
        assert link.exchange(REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, EXECUTE, 2, 2, 0, *([0] * 4), *([0] * 4),
                                          1, 0, 0, 0, *([151645] * 4), 1, 0, 0, 0)).transport_status == 12
        # wrong magic, wrong version, unknown operation
        assert link.exchange(REQUEST.pack(0x1234, PROTOCOL_VERSION, EXECUTE, *([0] * 23))).transport_status == 69
        assert link.exchange(REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION + 1, EXECUTE,
                                          *([0] * 23))).transport_status == 69
        assert link.exchange(REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, 9, *([0] * 23))).transport_status == 71
        # the session still serves epochs
        out = eng.execute(plan_of(request(0, 1, 5, 0), steps=2))
        assert out.token_ids == {"r0": [6, 7]}
        # an engine-side rejection (the double's 35 for a zero IPC magic) is an
        # error in PREPARED state: nothing reached the device
        with pytest.raises(ResidentEpochExecutionError) as err:
            eng._run(ResidentEpochPlan(CONTRACT_VERSION, 4, 1, 8, (request(0, 1, 5, 0),), (1, 0, 0, 0)),
                     DEVICE_IPC_EXECUTE, 3, b"\0" * IPC_METADATA_BYTES, "device_ipc")
        assert err.value.status == 35 and err.value.commit_state == EpochCommitState.PREPARED
    finally:
        eng.close()
    assert eng.process.returncode == 0


def test_startup_failure_reports_the_create_status(sidecar_env, monkeypatch):
    monkeypatch.setenv("STUB_CREATE_STATUS", "3")
    with pytest.raises(RuntimeError, match="native initialization failed: 103"):
        SidecarDataFlowEngine()


def test_startup_refuses_an_engine_that_is_not_four_rows(sidecar_env, monkeypatch):
    # the wire records hold four rows; a B=64 engine would overrun them
    monkeypatch.setenv("STUB_BATCH", "64")
    with pytest.raises(RuntimeError, match="native initialization failed: 101"):
        SidecarDataFlowEngine()
    log = Path(os.environ["STUB_LOG"]).read_text().splitlines()
    assert log[0].startswith("create ") and log[-1] == "destroy"


def test_server_exits_when_the_client_goes_away(sidecar_env):
    eng = SidecarDataFlowEngine()
    eng.link.close()
    eng.link = None
    assert eng.process.wait(timeout=30) == 68
    eng.close(force=True)


def test_server_rejects_a_socket_outside_dev_shm(stub_server, tmp_path):
    rc = subprocess.run([str(stub_server), str(tmp_path / "s.sock"), "a", "b", "c", "d", "e"]).returncode
    assert rc == 65
    assert subprocess.run([str(stub_server)]).returncode == 64


def test_in_process_engine_decodes_like_the_sidecar(sidecar_env, stub_server, monkeypatch):
    """The ctypes engine over the same C-ABI double returns what the sidecar
    returns for the same plans: both go through one feed/fetch codec."""
    monkeypatch.setenv("VLLM_ASCEND_RESIDENT_EPOCH_LIBRARY", str(stub_server.parent / "libresident_epoch.so"))
    plans = [plan_of(request(0, 1, 100, 0), request(2, 2, 200, 3)), plan_of(request(3, 4, 9, 5), steps=2)]
    local = CtypesDataFlowEngine()
    try:
        warm_local = local.warm_up()
        out_local = [local.execute(p) for p in plans]
        snap = small_snapshot(0b0010, (0, 5, 0, 0))
        imported = local.execute_with_import(plan_of(request(1, 5, 7, 2, imp=True), steps=2), snap)
    finally:
        local.close()
    assert imported.kv_imported and imported.kv_import_checksum == snap.checksum
    assert imported.kv_transfer_mode == "host_snapshot" and imported.token_ids == {"r1": [8, 9]}
    remote = SidecarDataFlowEngine()
    try:
        assert remote.warm_up() == warm_local
        assert [remote.execute(p) for p in plans] == out_local
    finally:
        remote.close()
    assert out_local[0].token_ids == {"r0": [101, 102, 103, 104], "r2": [201, 202, 203, 204]}
