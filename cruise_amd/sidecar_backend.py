"""Sidecar engine: the resident epoch served by ``resident_epoch_server`` in a
process of its own, driven over a Unix stream socket.

Interface kept from src/vllm_ascend_resident_epoch/sidecar_backend.py so the
reference's worker configuration works unchanged:

* the wire records (protocol 7): a 136-byte request ``<IHHiiQ4q4q4i4i4i``
  (magic 0x71317131, version, operation, request count, K, transfer id, then
  token/position/length/EOS/generation per row) and a 352-byte response
  ``<Iiiiiiii4q4i4i32q`` (magic 0x71327132, transport status, device status,
  model calls, feeds, fetches, commit state, checksum, wall/CPU microseconds,
  declared bytes, executed and generations per row, token history), with
  operations 1 execute, 2 warm-up, 3 shutdown, 4 import-execute, 5
  device-IPC execute (whose request is followed by the 4,088-byte IPC
  record) (sidecar_backend.py:23-36);
* the startup handshake: the server answers a response with transport
  status 0, or 100 + its create status, before taking requests;
* the environment: VLLM_ASCEND_RESIDENT_EPOCH_{SERVER, AIR, GRAPH_CONFIG,
  FUNC_CONFIG, TILING, EXTERNAL_WEIGHTS, SOCKET, CHILD_LIBRARY_PATH,
  STARTUP_TIMEOUT}; the socket, the weights and the KV transfer file live
  under /dev/shm.  SERVER defaults to the server built into this package.
  The Ascend-only child settings (custom operator path, memcpy trace
  preload) have no counterpart on this platform and are not read.

Structure: ``SidecarLaunch`` resolves the environment into a launch
description, ``SidecarLink`` frames records over the socket, and
``SidecarDataFlowEngine`` spawns the server and turns plans into records
through the shared feed/fetch codec (epoch_io.py).  Any failure between
sending a request and reading its whole answer is EXECUTING: the device may
or may not have run.
"""
from __future__ import annotations

import os
import socket
import struct
import subprocess
import time
from dataclasses import dataclass
from pathlib import Path

from .backend import NativeEpochOutput, NativeWarmupOutput
from .contract import EpochCommitState, ResidentEpochExecutionError, ResidentEpochPlan
from .epoch_io import (
    DEFAULT_EOS,
    MAX_EPOCH_STEPS,
    ROWS,
    WARMUP_GENERATION,
    WARMUP_TOKEN,
    EpochFeed,
    EpochFetch,
    check_transfer,
)
from .kv_transfer import IPC_METADATA_BYTES, DeviceKVTransfer, ResidentKVSnapshot, write_kv_snapshot
from .version import SIDECAR_PROTOCOL_VERSION

REQUEST_MAGIC = 0x71317131
RESPONSE_MAGIC = 0x71327132
PROTOCOL_VERSION = SIDECAR_PROTOCOL_VERSION
EXECUTE, WARM_UP, SHUTDOWN, IMPORT_EXECUTE, DEVICE_IPC_EXECUTE = 1, 2, 3, 4, 5
GRAPH_BATCH_SIZE = ROWS
REQUEST = struct.Struct("<IHHiiQ4q4q4i4i4i")
RESPONSE = struct.Struct("<Iiiiiiii4q4i4i32q")

DEFAULT_SERVER = Path(__file__).resolve().parent / "lib" / "resident_epoch_server"
SHM = "/dev/shm/"
ENV = "VLLM_ASCEND_RESIDENT_EPOCH_"

__all__ = [
    "DEFAULT_EOS", "DEVICE_IPC_EXECUTE", "EXECUTE", "GRAPH_BATCH_SIZE", "IMPORT_EXECUTE", "MAX_EPOCH_STEPS",
    "PROTOCOL_VERSION", "REQUEST", "REQUEST_MAGIC", "RESPONSE", "RESPONSE_MAGIC", "SHUTDOWN", "WARMUP_GENERATION",
    "WARMUP_TOKEN", "WARM_UP", "SidecarDataFlowEngine", "SidecarLaunch", "SidecarLink", "create_sidecar_engine",
    "decode_response", "encode_request",
]


def encode_request(operation: int, feed: EpochFeed, transfer_id: int = 0) -> bytes:
    return REQUEST.pack(REQUEST_MAGIC, PROTOCOL_VERSION, operation, feed.request_count, feed.max_steps, transfer_id,
                        *feed.tokens, *feed.positions, *feed.lengths, *feed.eos, *feed.generations)


def decode_response(record: bytes) -> EpochFetch:
    v = RESPONSE.unpack(record)
    if v[0] != RESPONSE_MAGIC:
        raise RuntimeError(f"sidecar response starts with {v[0]:#010x}, not the response magic")
    return EpochFetch(
        transport_status=v[1], device_status=v[2], model_calls=v[3], feed_calls=v[4], fetch_calls=v[5],
        commit_code=v[6], checksum=v[7], wall_us=v[8], native_cpu_us=v[9], declared_input_bytes=v[10],
        declared_output_bytes=v[11], executed=tuple(v[12:16]), generations=tuple(v[16:20]),
        history=tuple(v[20:20 + ROWS * MAX_EPOCH_STEPS]), source="resident epoch sidecar",
    )


def _existing(name: str, *, directory: bool = False, default: Path | None = None) -> Path:
    raw = os.getenv(ENV + name)
    if not raw and default is None:
        raise RuntimeError(f"{ENV}{name} must be set for the resident epoch sidecar")
    path = Path(raw).resolve() if raw else default
    if not (path.is_dir() if directory else path.is_file()):
        raise RuntimeError(f"{ENV}{name}: {path} is not an existing {'directory' if directory else 'file'}")
    return path


@dataclass(frozen=True)
class SidecarLaunch:
    """Everything needed to start the server: its argv (socket, then the
    five create arguments), its environment and the startup timeout."""

    server: Path
    socket_path: Path
    create_args: tuple[Path, ...]
    env: dict
    startup_timeout: float

    @property
    def transfer_path(self) -> Path:
        """The host-snapshot file of import-execute requests, beside the
        socket."""
        return self.socket_path.with_name(self.socket_path.name + ".kv-transfer")

    @property
    def argv(self) -> list[str]:
        return [str(self.server), str(self.socket_path), *map(str, self.create_args)]

    @classmethod
    def from_env(cls) -> "SidecarLaunch":
        server = _existing("SERVER", default=DEFAULT_SERVER)
        create_args = (_existing("AIR"), _existing("GRAPH_CONFIG"), _existing("FUNC_CONFIG"),
                       _existing("EXTERNAL_WEIGHTS", directory=True), _existing("TILING"))
        raw_socket = os.getenv(ENV + "SOCKET")
        if not raw_socket:
            raise RuntimeError(f"{ENV}SOCKET must name the sidecar's socket")
        socket_path = Path(raw_socket).resolve()
        env = dict(os.environ)
        extra = os.getenv(ENV + "CHILD_LIBRARY_PATH")
        if extra:
            roots = [Path(p).resolve() for p in extra.split(":")]
            missing = [str(p) for p in roots if not p.is_dir()]
            if missing:
                raise RuntimeError(f"{ENV}CHILD_LIBRARY_PATH names missing directories: {missing}")
            env["LD_LIBRARY_PATH"] = ":".join([*map(str, roots), *filter(None, [env.get("LD_LIBRARY_PATH")])])
        launch = cls(server, socket_path, create_args, env,
                     float(os.getenv(ENV + "STARTUP_TIMEOUT", "3600")))
        for what, path in (("socket", socket_path), ("external weight directory", create_args[3]),
                           ("KV transfer file", launch.transfer_path)):
            if not str(path).startswith(SHM):
                raise RuntimeError(f"the sidecar's {what} must be under {SHM}, got {path}")
        return launch


class SidecarLink:
    """A connected control socket carrying whole records."""

    def __init__(self, sock: socket.socket, peer: subprocess.Popen) -> None:
        self.sock = sock
        self.peer = peer

    @classmethod
    def connect(cls, path: Path, peer: subprocess.Popen, deadline: float) -> "SidecarLink | None":
        """Connect once the server listens; None at the deadline.  Raises if
        the server exits first."""
        while time.monotonic() < deadline:
            if peer.poll() is not None:
                raise RuntimeError(f"the resident epoch sidecar exited during startup with status {peer.returncode}")
            if path.exists():
                sock = socket.socket(socket.AF_UNIX, socket.SOCK_STREAM)
                try:
                    sock.connect(str(path))
                    return cls(sock, peer)
                except OSError:
                    sock.close()
            time.sleep(0.05)
        return None

    def read_record(self) -> EpochFetch:
        data = bytearray()
        while len(data) < RESPONSE.size:
            chunk = self.sock.recv(RESPONSE.size - len(data))
            if not chunk:
                raise RuntimeError(f"the resident epoch sidecar closed its socket (server status {self.peer.poll()})")
            data += chunk
        return decode_response(bytes(data))

    def exchange(self, record: bytes) -> EpochFetch:
        self.sock.sendall(record)
        return self.read_record()

    def close(self) -> None:
        self.sock.close()


class SidecarDataFlowEngine:
    """Starts the server, waits for its startup response, then serves the
    NativeEpochEngine protocol over the socket."""

    warmup_token = WARMUP_TOKEN
    warmup_eos = DEFAULT_EOS

    def __init__(self) -> None:
        self.launch = SidecarLaunch.from_env()
        self.socket_path = self.launch.socket_path
        self.transfer_path = self.launch.transfer_path
        self._remove_files(strict=True)
        self.link: SidecarLink | None = None
        self.process = subprocess.Popen(self.launch.argv, close_fds=True, env=self.launch.env)
        self.link = SidecarLink.connect(self.socket_path, self.process,
                                        time.monotonic() + self.launch.startup_timeout)
        if self.link is None:
            self._stop_process()
            raise TimeoutError(f"the resident epoch sidecar did not open {self.socket_path} in time")
        self.link.sock.settimeout(self.launch.startup_timeout)
        startup = self.link.read_record()
        if startup.transport_status != 0:
            self.close(force=True)
            raise RuntimeError(f"the sidecar's native initialization failed: {startup.transport_status}")

    # -- the engine protocol -------------------------------------------------
    def warm_up(self) -> NativeWarmupOutput:
        if self.link is None:
            raise RuntimeError("the resident epoch sidecar is closed")
        feed = EpochFeed.warm_up(self.warmup_token, self.warmup_eos)
        return self.link.exchange(encode_request(WARM_UP, feed)).warmup_output()

    def execute(self, plan: ResidentEpochPlan) -> NativeEpochOutput:
        return self._run(plan, EXECUTE, 0, b"", "none")

    def execute_with_import(self, plan: ResidentEpochPlan, snapshot: ResidentKVSnapshot) -> NativeEpochOutput:
        snapshot.validate()
        check_transfer(plan, snapshot.import_mask, snapshot.row_generations, "KV snapshot")
        write_kv_snapshot(self.transfer_path, snapshot)
        try:
            return self._run(plan, IMPORT_EXECUTE, snapshot.transfer_id, b"", "host_snapshot")
        finally:
            self.transfer_path.unlink(missing_ok=True)

    def execute_with_device_transfer(self, plan: ResidentEpochPlan, transfer: DeviceKVTransfer) -> NativeEpochOutput:
        transfer.validate()
        check_transfer(plan, transfer.import_mask, transfer.row_generations, "device KV transfer")
        record = transfer.wire_bytes()
        if len(record) != IPC_METADATA_BYTES:
            raise ValueError(f"a device IPC record is {IPC_METADATA_BYTES} bytes, not {len(record)}")
        return self._run(plan, DEVICE_IPC_EXECUTE, transfer.transfer_id, record, "device_ipc")

    def _run(self, plan: ResidentEpochPlan, operation: int, transfer_id: int, trailer: bytes,
             mode: str) -> NativeEpochOutput:
        if self.link is None:
            raise ResidentEpochExecutionError("the resident epoch sidecar is closed",
                                              commit_state=EpochCommitState.PREPARED)
        record = encode_request(operation, EpochFeed.from_plan(plan), transfer_id) + trailer
        try:
            fetch = self.link.exchange(record)
        except Exception as exc:
            raise ResidentEpochExecutionError(f"no complete answer from the sidecar: {exc}",
                                              commit_state=EpochCommitState.EXECUTING) from exc
        return fetch.native_output(plan, mode)

    # -- lifecycle -----------------------------------------------------------
    def _remove_files(self, strict: bool = False) -> None:
        for path in (self.socket_path, self.transfer_path):
            try:
                path.unlink(missing_ok=True)
            except OSError as exc:
                if strict:
                    raise RuntimeError(f"cannot remove the stale sidecar file {path}: {exc}") from exc

    def _stop_process(self) -> None:
        """Terminate, then kill, waiting up to a minute for each."""
        for signal_process in (self.process.terminate, self.process.kill):
            if self.process.poll() is not None:
                return
            signal_process()
            try:
                self.process.wait(timeout=60)
                return
            except subprocess.TimeoutExpired:
                continue

    def close(self, *, force: bool = False) -> None:
        """Ask a running server to shut down; if that fails, or with
        ``force``, stop its process instead."""
        if self.link is not None:
            if not force and self.process.poll() is None:
                try:
                    self.link.exchange(encode_request(SHUTDOWN, EpochFeed.empty()))
                except (OSError, RuntimeError):
                    force = True
            self.link.close()
            self.link = None
        if not force:
            try:
                self.process.wait(timeout=300)
            except subprocess.TimeoutExpired:
                force = True
        if force:
            self._stop_process()
        self._remove_files()

    def __del__(self) -> None:
        try:
            if getattr(self, "process", None) is not None:
                self.close(force=True)
        except Exception:
            pass


def create_sidecar_engine() -> SidecarDataFlowEngine:
    return SidecarDataFlowEngine()
