"""Sidecar engine: the resident epoch served by ``resident_epoch_server`` in
its own process, driven over a Unix socket.

Mirrors src/vllm_ascend_resident_epoch/sidecar_backend.py:23-466: the same
environment variables, wire records (136-byte request ``<IHHiiQ4q4q4i4i4i``,
352-byte response ``<Iiiiiiii4q4i4i32q``, protocol 7), operations, warm-up
request, startup handshake and shutdown escalation.  The server binary
defaults to the one built into this package (cruise_amd/lib/
resident_epoch_server) when VLLM_ASCEND_RESIDENT_EPOCH_SERVER is unset.
The reference's Ascend-only child settings (custom operator path, memcpy
trace preload) have no MI355X counterpart and are not read.
"""
from __future__ import annotations

import os
import socket
import struct
import subprocess
import time
from pathlib import Path

from .backend import NativeEpochOutput, NativeWarmupOutput
from .contract import EpochCommitState, ResidentEpochExecutionError, ResidentEpochPlan
from .kv_transfer import IPC_METADATA_BYTES, DeviceKVTransfer, ResidentKVSnapshot, write_kv_snapshot
from .version import SIDECAR_PROTOCOL_VERSION

REQUEST_MAGIC = 0x71317131
RESPONSE_MAGIC = 0x71327132
PROTOCOL_VERSION = SIDECAR_PROTOCOL_VERSION
EXECUTE = 1
WARM_UP = 2
SHUTDOWN = 3
IMPORT_EXECUTE = 4
DEVICE_IPC_EXECUTE = 5
GRAPH_BATCH_SIZE = 4
MAX_EPOCH_STEPS = 8
WARMUP_GENERATION = 2**31 - 1
WARMUP_TOKEN = 11690
DEFAULT_EOS = 151645
REQUEST = struct.Struct("<IHHiiQ4q4q4i4i4i")
RESPONSE = struct.Struct("<Iiiiiiii4q4i4i32q")

DEFAULT_SERVER = Path(__file__).resolve().parent / "lib" / "resident_epoch_server"

# Response field positions (RESPONSE.unpack order).
_TRANSPORT, _DEVICE, _CALLS, _FEEDS, _FETCHES, _COMMIT, _CHECKSUM = 1, 2, 3, 4, 5, 6, 7
_WALL, _CPU, _IN_BYTES, _OUT_BYTES = 8, 9, 10, 11
_EXECUTED = slice(12, 16)
_GENERATIONS = slice(16, 20)
_TOKENS = slice(20, 20 + GRAPH_BATCH_SIZE * MAX_EPOCH_STEPS)


def _commit_state(value: int) -> EpochCommitState:
    try:
        return EpochCommitState(value)
    except ValueError as exc:
        raise ResidentEpochExecutionError(
            f"sidecar returned invalid commit state {value}", commit_state=EpochCommitState.EXECUTING
        ) from exc


def _env_path(name: str, *, directory: bool = False, default: Path | None = None) -> Path:
    raw = os.getenv(name)
    if not raw and default is None:
        raise RuntimeError(f"{name} is required by the resident epoch sidecar")
    path = Path(raw).resolve() if raw else default
    if not (path.is_dir() if directory else path.is_file()):
        raise RuntimeError(f"{name} must name an existing {'directory' if directory else 'file'}: {path}")
    return path


def _by_row(plan: ResidentEpochPlan, field: str, fill: int) -> list[int]:
    values = [fill] * GRAPH_BATCH_SIZE
    for r in plan.requests:
        values[r.row] = int(getattr(r, field))
    return values


def _request(operation: int, count: int, steps: int, transfer_id: int, tokens, positions, lengths, eos, gens) -> bytes:
    return REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, operation, count, steps, transfer_id,
                        *tokens, *positions, *lengths, *eos, *gens)


class SidecarDataFlowEngine:
    """Spawns the server, waits for its startup response, then runs epochs."""

    warmup_token = WARMUP_TOKEN
    warmup_eos = DEFAULT_EOS

    def __init__(self) -> None:
        server = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_SERVER", default=DEFAULT_SERVER)
        air = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_AIR")
        graph_config = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_GRAPH_CONFIG")
        func_config = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_FUNC_CONFIG")
        tiling = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_TILING")
        weights = _env_path("VLLM_ASCEND_RESIDENT_EPOCH_EXTERNAL_WEIGHTS", directory=True)
        raw_socket = os.getenv("VLLM_ASCEND_RESIDENT_EPOCH_SOCKET")
        if not raw_socket:
            raise RuntimeError("VLLM_ASCEND_RESIDENT_EPOCH_SOCKET is required")
        self.socket_path = Path(raw_socket).resolve()
        self.transfer_path = self.socket_path.with_name(self.socket_path.name + ".kv-transfer")
        for what, p in (("socket", self.socket_path), ("external weights", weights), ("KV transfer file", self.transfer_path)):
            if not str(p).startswith("/dev/shm/"):
                raise RuntimeError(f"resident epoch {what} must be under /dev/shm")

        env = os.environ.copy()
        extra_libs = os.getenv("VLLM_ASCEND_RESIDENT_EPOCH_CHILD_LIBRARY_PATH")
        if extra_libs:
            roots = [Path(p).resolve() for p in extra_libs.split(":")]
            if not all(p.is_dir() for p in roots):
                raise RuntimeError("resident sidecar library path is invalid")
            inherited = env.get("LD_LIBRARY_PATH")
            env["LD_LIBRARY_PATH"] = ":".join([*map(str, roots), *([inherited] if inherited else [])])

        try:
            self.socket_path.unlink(missing_ok=True)
            self.transfer_path.unlink(missing_ok=True)
        except OSError as exc:
            raise RuntimeError(f"cannot reset sidecar socket: {exc}") from exc
        argv = [str(server), str(self.socket_path), str(air), str(graph_config), str(func_config), str(weights), str(tiling)]
        self.process = subprocess.Popen(argv, close_fds=True, env=env)
        self.socket: socket.socket | None = None
        timeout = int(os.getenv("VLLM_ASCEND_RESIDENT_EPOCH_STARTUP_TIMEOUT", "3600"))
        self.socket = self._connect(time.monotonic() + timeout)
        if self.socket is None:
            self._stop_process()
            raise TimeoutError("resident epoch sidecar socket startup timed out")
        self.socket.settimeout(timeout)
        startup = self._receive_response()
        if startup[_TRANSPORT] != 0:
            status = startup[_TRANSPORT]
            self.close(force=True)
            raise RuntimeError(f"resident epoch sidecar native initialization failed: {status}")

    def _connect(self, deadline: float) -> socket.socket | None:
        while time.monotonic() < deadline:
            if self.process.poll() is not None:
                raise RuntimeError(f"resident epoch sidecar exited during startup with status {self.process.returncode}")
            if self.socket_path.exists():
                s = socket.socket(socket.AF_UNIX, socket.SOCK_STREAM)
                try:
                    s.connect(str(self.socket_path))
                    return s
                except OSError:
                    s.close()
            time.sleep(0.05)
        return None

    # -- wire ------------------------------------------------------------------
    def _receive_exact(self, size: int) -> bytes:
        assert self.socket is not None
        buf = bytearray()
        while len(buf) < size:
            chunk = self.socket.recv(size - len(buf))
            if not chunk:
                raise RuntimeError(f"resident epoch sidecar closed the control socket (status={self.process.poll()})")
            buf += chunk
        return bytes(buf)

    def _receive_response(self) -> tuple[int, ...]:
        values = RESPONSE.unpack(self._receive_exact(RESPONSE.size))
        if values[0] != RESPONSE_MAGIC:
            raise RuntimeError("resident epoch sidecar response magic mismatch")
        return values

    # -- operations --------------------------------------------------------------
    def warm_up(self) -> NativeWarmupOutput:
        """One decoder step of one row under the reserved generation
        (sidecar_backend.py:218-272)."""
        if self.socket is None:
            raise RuntimeError("resident epoch sidecar is closed")
        self.socket.sendall(
            _request(WARM_UP, 1, 1, 0, [self.warmup_token, 0, 0, 0], [0] * 4, [1, 0, 0, 0],
                     [self.warmup_eos] * 4, [WARMUP_GENERATION, 0, 0, 0])
        )
        v = self._receive_response()
        commit = _commit_state(v[_COMMIT])
        if v[_TRANSPORT] != 0:
            raise ResidentEpochExecutionError(
                f"resident epoch warmup failed: {v[_TRANSPORT]}", commit_state=commit, status=v[_TRANSPORT]
            )
        if v[_EXECUTED] != (1, 0, 0, 0):
            raise RuntimeError("resident epoch warmup did not execute exactly one row")
        if v[_GENERATIONS] != (WARMUP_GENERATION, 0, 0, 0):
            raise RuntimeError("resident epoch warmup generation acknowledgement failed")
        return NativeWarmupOutput(
            status=v[_DEVICE], model_calls=v[_CALLS], feed_calls=v[_FEEDS], fetch_calls=v[_FETCHES],
            commit_state=commit, wall_us=v[_WALL], native_cpu_us=v[_CPU],
            declared_input_bytes=v[_IN_BYTES], declared_output_bytes=v[_OUT_BYTES],
        )

    def execute(self, plan: ResidentEpochPlan) -> NativeEpochOutput:
        return self._execute(plan, operation=EXECUTE, transfer_id=0)

    @staticmethod
    def _import_check(plan: ResidentEpochPlan, mask: int, generations, what: str) -> None:
        rows = [r for r in plan.requests if r.kv_import_required]
        if mask != sum(1 << r.row for r in rows):
            raise ValueError(f"{what} mask does not match the resident plan")
        expected = [0] * GRAPH_BATCH_SIZE
        for r in rows:
            expected[r.row] = r.generation
        if tuple(generations) != tuple(expected):
            raise ValueError(f"{what} generations do not match the resident plan")

    def execute_with_import(self, plan: ResidentEpochPlan, snapshot: ResidentKVSnapshot) -> NativeEpochOutput:
        snapshot.validate()
        self._import_check(plan, snapshot.import_mask, snapshot.row_generations, "KV snapshot")
        write_kv_snapshot(self.transfer_path, snapshot)
        try:
            return self._execute(plan, operation=IMPORT_EXECUTE, transfer_id=snapshot.transfer_id)
        finally:
            self.transfer_path.unlink(missing_ok=True)

    def execute_with_device_transfer(self, plan: ResidentEpochPlan, transfer: DeviceKVTransfer) -> NativeEpochOutput:
        transfer.validate()
        self._import_check(plan, transfer.import_mask, transfer.row_generations, "device KV transfer")
        return self._execute(plan, operation=DEVICE_IPC_EXECUTE, transfer_id=transfer.transfer_id,
                             ipc_metadata=transfer.wire_bytes())

    def _execute(self, plan: ResidentEpochPlan, *, operation: int, transfer_id: int,
                 ipc_metadata: bytes | None = None) -> NativeEpochOutput:
        if self.socket is None:
            raise ResidentEpochExecutionError("resident epoch sidecar is closed", commit_state=EpochCommitState.PREPARED)
        if plan.graph_batch_size != GRAPH_BATCH_SIZE:
            raise ValueError("the sidecar backend owns only the static B=4 graph")
        payload = _request(operation, len(plan.requests), plan.max_steps, transfer_id,
                           _by_row(plan, "token_id", 0), _by_row(plan, "position", 0),
                           _by_row(plan, "sequence_length", 0), _by_row(plan, "eos_token_id", DEFAULT_EOS),
                           plan.row_generations)
        if operation == DEVICE_IPC_EXECUTE:
            if ipc_metadata is None or len(ipc_metadata) != IPC_METADATA_BYTES:
                raise ValueError("direct Device KV operation has invalid metadata")
            payload += ipc_metadata
        try:
            self.socket.sendall(payload)
            v = self._receive_response()
        except Exception as exc:
            # The request may or may not have reached the device.
            raise ResidentEpochExecutionError(
                f"resident epoch response is ambiguous: {exc}", commit_state=EpochCommitState.EXECUTING
            ) from exc
        commit = _commit_state(v[_COMMIT])
        if v[_TRANSPORT] != 0:
            raise ResidentEpochExecutionError(
                f"resident epoch sidecar execute failed: {v[_TRANSPORT]}", commit_state=commit, status=v[_TRANSPORT]
            )
        executed = v[_EXECUTED]
        history = v[_TOKENS]
        tokens: dict[str, list[int]] = {}
        for r in plan.requests:
            n = executed[r.row]
            if not 0 <= n <= plan.max_steps:
                raise ResidentEpochExecutionError("sidecar returned an invalid executed count", commit_state=commit)
            tokens[r.req_id] = list(history[r.row * MAX_EPOCH_STEPS : r.row * MAX_EPOCH_STEPS + n])
        imported = operation in (IMPORT_EXECUTE, DEVICE_IPC_EXECUTE)
        return NativeEpochOutput(
            status=v[_DEVICE], model_calls=v[_CALLS], token_ids=tokens, row_generations=tuple(v[_GENERATIONS]),
            commit_state=commit, feed_calls=v[_FEEDS], fetch_calls=v[_FETCHES], wall_us=v[_WALL],
            native_cpu_us=v[_CPU], declared_input_bytes=v[_IN_BYTES], declared_output_bytes=v[_OUT_BYTES],
            kv_imported=imported, kv_import_checksum=v[_CHECKSUM] & 0xFFFFFFFF,
            kv_transfer_mode=("device_ipc" if operation == DEVICE_IPC_EXECUTE else "host_snapshot") if imported else "none",
        )

    # -- lifecycle ---------------------------------------------------------------
    def _stop_process(self) -> None:
        if self.process.poll() is None:
            self.process.terminate()
            try:
                self.process.wait(timeout=60)
            except subprocess.TimeoutExpired:
                self.process.kill()
                self.process.wait(timeout=60)

    def close(self, *, force: bool = False) -> None:
        """Graceful SHUTDOWN when the server still runs, else (or if that
        fails) terminate, then kill (sidecar_backend.py:416-456)."""
        if self.socket is not None:
            if not force and self.process.poll() is None:
                try:
                    self.socket.sendall(_request(SHUTDOWN, 0, 0, 0, [0] * 4, [0] * 4, [0] * 4, [0] * 4, [0] * 4))
                    self._receive_response()
                except (OSError, RuntimeError):
                    force = True
            self.socket.close()
            self.socket = None
        if force:
            self._stop_process()
        else:
            try:
                self.process.wait(timeout=300)
            except subprocess.TimeoutExpired:
                self._stop_process()
        for p in (self.socket_path, self.transfer_path):
            try:
                p.unlink(missing_ok=True)
            except OSError:
                pass

    def __del__(self) -> None:
        try:
            self.close(force=True)
        except Exception:
            pass


def create_sidecar_engine() -> SidecarDataFlowEngine:
    return SidecarDataFlowEngine()
