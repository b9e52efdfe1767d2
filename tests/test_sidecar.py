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


def test_warmup_request_uses_the_reserved_generation():
    sent = []

    class Recorder:
        def sendall(self, data):
            sent.append(data)

    eng = SidecarDataFlowEngine.__new__(SidecarDataFlowEngine)
    eng.socket = Recorder()
    eng._receive_response = lambda: RESPONSE.unpack(
        RESPONSE.pack(RESPONSE_MAGIC, 0, 0, 1, 1, 1, 2, 0, 7, 3, 260, 368, 1, 0, 0, 0,
                      WARMUP_GENERATION, 0, 0, 0, 12, *([-1] * 31))
    )
    out = eng.warm_up()
    fields = REQUEST.unpack(sent[0])
    assert fields[:5] == (REQUEST_MAGIC, PROTOCOL_VERSION, WARM_UP, 1, 1)
    assert fields[6:10] == (11690, 0, 0, 0)
    assert fields[-GRAPH_BATCH_SIZE:] == (WARMUP_GENERATION, 0, 0, 0)
    assert (out.status, out.model_calls, out.feed_calls, out.fetch_calls) == (0, 1, 1, 1)


def test_device_ipc_execute_is_reported_as_kv_import():
    sent = []

    class Recorder:
        def sendall(self, data):
            sent.append(data)

    eng = SidecarDataFlowEngine.__new__(SidecarDataFlowEngine)
    eng.socket = Recorder()
    eng._receive_response = lambda: RESPONSE.unpack(
        RESPONSE.pack(RESPONSE_MAGIC, 0, 0, 1, 1, 1, EpochCommitState.COMMITTED, 0x12345678, 123, 45, 3776, 368,
                      1, 0, 0, 0, 7, 0, 0, 0, 42, *([-1] * 31))
    )
    plan = plan_of(request(0, 7, 11, 1, imp=True), steps=1)
    metadata = b"\0" * IPC_METADATA_BYTES
    out = eng._execute(plan, operation=DEVICE_IPC_EXECUTE, transfer_id=9, ipc_metadata=metadata)
    assert out.kv_imported is True
    assert out.kv_import_checksum == 0x12345678
    assert out.token_ids == {"r0": [42]}
    assert len(sent) == 1 and sent[0][REQUEST.size:] == metadata
    assert REQUEST.unpack(sent[0][: REQUEST.size])[2] == DEVICE_IPC_EXECUTE


def test_invalid_commit_state_is_ambiguous():
    eng = SidecarDataFlowEngine.__new__(SidecarDataFlowEngine)
    eng.socket = type("S", (), {"sendall": lambda self, d: None})()
    eng._receive_response = lambda: RESPONSE.unpack(
        RESPONSE.pack(RESPONSE_MAGIC, 0, 0, 1, 1, 1, 9, 0, 0, 0, 0, 0, *([0] * 8), *([-1] * 32))
    )
    with pytest.raises(ResidentEpochExecutionError) as err:
        eng.execute(plan_of(request(0, 1, 5, 0)))
    assert err.value.commit_state == EpochCommitState.EXECUTING


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
        eng.socket.sendall(REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, EXECUTE, 2, 2, 0, *([0] * 4), *([0] * 4),
                                        1, 0, 0, 0, *([151645] * 4), 1, 0, 0, 0))
        assert eng._receive_response()[1] == 12
        # wrong magic, wrong version, unknown operation
        eng.socket.sendall(REQUEST.pack(0x1234, PROTOCOL_VERSION, EXECUTE, *([0] * 23)))
        assert eng._receive_response()[1] == 69
        eng.socket.sendall(REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION + 1, EXECUTE, *([0] * 23)))
        assert eng._receive_response()[1] == 69
        eng.socket.sendall(REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, 9, *([0] * 23)))
        assert eng._receive_response()[1] == 71
        # the session still serves epochs
        out = eng.execute(plan_of(request(0, 1, 5, 0), steps=2))
        assert out.token_ids == {"r0": [6, 7]}
        # an engine-side rejection (the double's 35 for a zero IPC magic) is an
        # error in PREPARED state: nothing reached the device
        with pytest.raises(ResidentEpochExecutionError) as err:
            eng._execute(ResidentEpochPlan(CONTRACT_VERSION, 4, 1, 8, (request(0, 1, 5, 0),), (1, 0, 0, 0)),
                         operation=DEVICE_IPC_EXECUTE, transfer_id=3, ipc_metadata=b"\0" * IPC_METADATA_BYTES)
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
    eng.socket.close()
    eng.socket = None
    assert eng.process.wait(timeout=30) == 68
    eng.close(force=True)


def test_server_rejects_a_socket_outside_dev_shm(stub_server, tmp_path):
    rc = subprocess.run([str(stub_server), str(tmp_path / "s.sock"), "a", "b", "c", "d", "e"]).returncode
    assert rc == 65
    assert subprocess.run([str(stub_server)]).returncode == 64
