"""Python runtime over the C-ABI of libresident_epoch.so.

``ResidentEpochRuntime`` owns one engine (the library keeps the reference's
process-wide singleton, native/resident_epoch_bridge.cpp:94-95, 366-371) and
exposes the three levels of the reference's interface:

* ``execute``       -- the bridge call ``resident_epoch_execute`` (host rows in,
  per-row tokens out; resident_epoch_bridge.cpp:424-649);
* ``proc``          -- the 8-input/2-output epoch ABI (``G4cB4ResidentEpoch::Proc``);
* ``decoder_step``  -- the 9-input/4-output decoder ABI (``PagedQwenDecoderStep``).

Tensors may be numpy arrays or torch tensors (CPU or GPU); they are handed to
the library as plain pointers.
"""
from __future__ import annotations

import ctypes
import json
import os
import shutil
import tempfile
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

from . import _lib

MAX_EPOCH_STEPS = 8
TILING_WORDS = (28, 1, 128, 8, 16, 512, 16, 1, 1, 1, 28, 5, 2336, 24, 0, 0, 0, 0)  # batched_decoder_step.py:36


def tiling_bytes() -> bytes:
    """The 72-byte ExactQk tiling record the reference feeds (kept for ABI
    compatibility; the HIP kernels do not read it)."""
    return np.asarray(TILING_WORDS, dtype="<u4").tobytes()


@dataclass(frozen=True)
class ModelSpec:
    num_layers: int = 28
    hidden: int = 3584
    num_heads: int = 28
    num_kv_heads: int = 4
    head_dim: int = 128
    intermediate: int = 18944
    vocab: int = 152064
    rope_theta: float = 1_000_000.0
    rms_eps: float = 1e-6
    dtype: str = "bf16"


@dataclass(frozen=True)
class EngineSpec:
    batch: int = 4
    physical_blocks: int = 8
    block_size: int = 128
    blocks_per_row: int = 2
    logical_capacity: int = 8
    configured_eos: int = 151645
    require_dev_shm: bool = True


@dataclass(frozen=True)
class WeightSpec:
    source: str = "upload"  # "bundle" | "synthetic" | "upload"
    seed: int = 0
    std: float = 0.02


@dataclass(frozen=True)
class EngineConfig:
    model: ModelSpec = field(default_factory=ModelSpec)
    engine: EngineSpec = field(default_factory=EngineSpec)
    weights: WeightSpec = field(default_factory=WeightSpec)
    # Launch-plan selections that cross-check alternative kernels of the
    # same arithmetic (for example {"attention_split": 1}); the keys are
    # listed where the engine reads them.
    tuning: dict = field(default_factory=dict)

    def to_json(self) -> str:
        doc = {"model": asdict(self.model), "engine": asdict(self.engine), "weights": asdict(self.weights)}
        if self.tuning:
            doc["tuning"] = dict(self.tuning)
        return json.dumps(doc)


def _ptr(value: Any) -> tuple[int, Any]:
    """(address, keep-alive) of a numpy array or torch tensor."""
    if value is None:
        return 0, None
    try:
        import torch

        if isinstance(value, torch.Tensor):
            t = value.contiguous()
            if t.is_cuda:
                torch.cuda.synchronize(t.device)
            return t.data_ptr(), t
    except ImportError:  # pragma: no cover - torch is present in this image
        pass
    arr = np.ascontiguousarray(value)
    return arr.ctypes.data, arr


def _nbytes(value: Any) -> int:
    try:
        import torch

        if isinstance(value, torch.Tensor):
            return value.numel() * value.element_size()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(value).nbytes


def feed_layout(batch: int, blocks_per_row: int, importing: bool = False, payload_bytes: int = 0) -> dict[str, tuple[int, int]]:
    """Byte offsets/sizes of the packed epoch feed (native/resident_epoch_bridge.cpp:53-62)."""
    off = payload_bytes if importing else 0
    out = {}
    if importing:
        out["payload"] = (0, payload_bytes)
    for name, size in (
        ("token", 8 * batch),
        ("position", 8 * batch),
        ("sequence_length", 4 * batch),
        ("slot_mapping", 0 if importing else 4 * batch),
        ("active_mask", 4 * batch),
        ("block_table", 4 * batch * blocks_per_row),
        ("tiling", 72),
        ("control", 4 * (3 + 2 * batch)),
    ):
        if size:
            out[name] = (off, size)
        off += size
    out["_total"] = (0, off)
    return out


def pack_feed(
    token, position, sequence_length, slot_mapping, active_mask, block_table, tiling: bytes, control, payload: bytes | None = None
) -> bytes:
    parts = []
    if payload is not None:
        parts.append(bytes(payload))
    parts.append(np.asarray(token, dtype="<i8").reshape(-1).tobytes())
    parts.append(np.asarray(position, dtype="<i8").reshape(-1).tobytes())
    parts.append(np.asarray(sequence_length, dtype="<i4").reshape(-1).tobytes())
    if payload is None:
        parts.append(np.asarray(slot_mapping, dtype="<i4").reshape(-1).tobytes())
    parts.append(np.asarray(active_mask, dtype="<i4").reshape(-1).tobytes())
    parts.append(np.asarray(block_table, dtype="<i4").reshape(-1).tobytes())
    if len(tiling) != 72:
        raise ValueError("tiling must be 72 bytes")
    parts.append(bytes(tiling))
    parts.append(np.asarray(control, dtype="<i4").reshape(-1).tobytes())
    return b"".join(parts)


def unpack_fetch(raw: bytes, batch: int) -> tuple[np.ndarray, np.ndarray]:
    hist = np.frombuffer(raw, dtype="<i8", count=MAX_EPOCH_STEPS * batch).reshape(MAX_EPOCH_STEPS, batch).copy()
    control = np.frombuffer(raw, dtype="<i4", offset=8 * MAX_EPOCH_STEPS * batch).copy()
    return hist, control


@dataclass
class BridgeOutput:
    status: int
    token_ids: np.ndarray  # [B, 8] int64
    executed: np.ndarray
    row_generations: np.ndarray
    model_calls: int
    device_status: int
    feed_calls: int
    fetch_calls: int
    commit_state: int
    kv_import_checksum: int
    wall_us: int
    native_cpu_us: int
    declared_input_bytes: int
    declared_output_bytes: int


class ResidentEpochRuntime:
    """One engine of libresident_epoch.so."""

    def __init__(
        self,
        config: EngineConfig,
        weights: dict[str, Any] | None = None,
        *,
        weight_dir: str | None = None,
        graph_config: str | None = None,
        workdir: str | None = None,
    ) -> None:
        self.lib = _lib.load()
        self.config = config
        base = "/dev/shm" if Path("/dev/shm").is_dir() else None
        self._workdir = Path(workdir or tempfile.mkdtemp(prefix="cruise-engine-", dir=base))
        self._owns_workdir = workdir is None
        cfg_path = Path(graph_config) if graph_config else self._workdir / "graph_config.json"
        if graph_config is None:
            cfg_path.write_text(config.to_json())
        tiling_path = self._workdir / "tiling.bin"
        tiling_path.write_bytes(tiling_bytes())
        wdir = weight_dir or str(self._workdir)
        status = ctypes.c_int32(-1)
        self.handle = self.lib.resident_epoch_create(
            b"unused.air",
            str(cfg_path).encode(),
            b"resident_epoch_func.json",
            wdir.encode(),
            str(tiling_path).encode(),
            ctypes.byref(status),
        )
        if not self.handle or status.value != 0:
            self._cleanup_dir()
            raise RuntimeError(f"resident_epoch_create failed, status={status.value}")
        self.batch = self.info("batch")
        self.vocab = self.info("vocab")
        self.blocks_per_row = self.info("blocks_per_row")
        self.feed_bytes = self.info("feed_bytes")
        self.import_feed_bytes = self.info("import_feed_bytes")
        self.fetch_bytes = self.info("fetch_bytes")
        self.cache_bytes = self.info("cache_bytes")
        if weights:
            for name, value in weights.items():
                self.write_state(name, value)

    # -- lifecycle ---------------------------------------------------------------
    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.resident_epoch_destroy(self.handle)
            self.handle = None
        self._cleanup_dir()

    def _cleanup_dir(self) -> None:
        if getattr(self, "_owns_workdir", False) and self._workdir.exists():
            shutil.rmtree(self._workdir, ignore_errors=True)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- state -------------------------------------------------------------------
    def info(self, key: str) -> int:
        value = ctypes.c_int64(0)
        if self.lib.resident_epoch_info(self.handle, key.encode(), ctypes.byref(value)) != 0:
            raise KeyError(key)
        return int(value.value)

    def write_state(self, name: str, value: Any) -> None:
        addr, keep = _ptr(value)
        rc = self.lib.resident_epoch_write_state(self.handle, name.encode(), addr, _nbytes(keep))
        if rc != 0:
            raise RuntimeError(f"write_state({name}) failed: {rc}")

    def read_state(self, name: str, out: Any) -> Any:
        addr, keep = _ptr(out)
        if keep is not out:
            raise ValueError("read_state needs a contiguous output buffer")
        rc = self.lib.resident_epoch_read_state(self.handle, name.encode(), addr, _nbytes(out))
        if rc != 0:
            raise RuntimeError(f"read_state({name}) failed: {rc}")
        return out

    def resident_rows(self) -> np.ndarray:
        rows = np.zeros((5, self.batch), dtype=np.int64)
        return self.read_state("resident_rows", rows)

    # -- ABIs --------------------------------------------------------------------
    def proc(self, feed: bytes) -> tuple[np.ndarray, np.ndarray]:
        """8-input/2-output epoch: one feed in, (history [8,B], control) out."""
        fetch = ctypes.create_string_buffer(self.fetch_bytes)
        feed_buf = ctypes.create_string_buffer(bytes(feed), len(feed))
        rc = self.lib.resident_epoch_proc(self.handle, feed_buf, len(feed), fetch, self.fetch_bytes)
        if rc != 0:
            raise RuntimeError(f"resident_epoch_proc failed: {rc}")
        return unpack_fetch(fetch.raw, self.batch)

    def decoder_step(self, token, position, sequence_length, key_cache, slot_mapping, active_mask, block_table, value_cache, logits, next_position, tiling=None):
        """9-input/4-output decoder step; key/value caches are updated in place."""
        tiling_arr = np.frombuffer(tiling or tiling_bytes(), dtype=np.uint8).copy()
        args = [token, position, sequence_length, key_cache, slot_mapping, active_mask, block_table, value_cache, tiling_arr, logits, next_position]
        ptrs = []
        keep = []
        for a in args:
            p, k = _ptr(a)
            ptrs.append(p)
            keep.append(k)
        for a, k in ((key_cache, keep[3]), (value_cache, keep[7]), (logits, keep[9]), (next_position, keep[10])):
            if k is not a:
                raise ValueError("output and cache buffers must be contiguous")
        rc = self.lib.resident_decoder_step(self.handle, *ptrs)
        if rc != 0:
            raise RuntimeError(f"resident_decoder_step failed: {rc}")

    def prefill(self, row: int, generation: int, prompt, block_table_row) -> None:
        p, kp = _ptr(np.asarray(prompt, dtype=np.int64))
        t, kt = _ptr(np.asarray(block_table_row, dtype=np.int32))
        rc = self.lib.resident_epoch_prefill(self.handle, row, generation, p, len(kp), t)
        if rc != 0:
            raise RuntimeError(f"resident_epoch_prefill failed: {rc}")

    def prefill_batch(self, rows, generations, prompts, block_tables, *, noalloc: bool = False) -> None:
        """Batched prefill of several rows at once (resident_epoch_prefill_batch,
        or with ``noalloc`` resident_epoch_prefill_batch_noalloc): ``prompts``
        is a list of token lists, ``block_tables`` [len(rows), BPR]."""
        lens = np.asarray([len(p) for p in prompts], dtype=np.int32)
        flat = np.concatenate([np.asarray(p, dtype=np.int64) for p in prompts]) if len(prompts) else np.zeros(0, np.int64)
        args = [np.asarray(rows, dtype=np.int32), np.asarray(generations, dtype=np.int32), flat, lens,
                np.ascontiguousarray(np.asarray(block_tables, dtype=np.int32))]
        ptrs = [_ptr(a) for a in args]
        name = "resident_epoch_prefill_batch_noalloc" if noalloc else "resident_epoch_prefill_batch"
        rc = getattr(self.lib, name)(self.handle, len(lens), *(p for p, _ in ptrs))
        if rc != 0:
            raise RuntimeError(f"{name} failed: {rc}")

    def execute(
        self,
        request_count: int,
        max_steps: int,
        tokens,
        positions,
        lengths,
        eos,
        generations,
        transfer_path: str | None = None,
        transfer_id: int = 0,
    ) -> BridgeOutput:
        B = self.batch
        i64 = ctypes.c_int64 * B
        i32 = ctypes.c_int32 * B
        out_tok = (ctypes.c_int64 * (B * MAX_EPOCH_STEPS))()
        out_exec = i32()
        out_gen = i32()
        scalars32 = [ctypes.c_int32(v) for v in (0, -1, 0, 0, -1, 0)]
        scalars64 = [ctypes.c_int64(0) for _ in range(4)]
        status = self.lib.resident_epoch_execute(
            self.handle,
            request_count,
            max_steps,
            i64(*[int(v) for v in tokens]),
            i64(*[int(v) for v in positions]),
            i32(*[int(v) for v in lengths]),
            i32(*[int(v) for v in eos]),
            i32(*[int(v) for v in generations]),
            out_tok,
            out_exec,
            out_gen,
            *[ctypes.byref(s) for s in scalars32],
            *[ctypes.byref(s) for s in scalars64],
            transfer_path.encode() if transfer_path else None,
            transfer_id,
            None,
        )
        return BridgeOutput(
            status=int(status),
            token_ids=np.frombuffer(out_tok, dtype=np.int64).reshape(B, MAX_EPOCH_STEPS).copy(),
            executed=np.frombuffer(out_exec, dtype=np.int32).copy(),
            row_generations=np.frombuffer(out_gen, dtype=np.int32).copy(),
            model_calls=scalars32[0].value,
            device_status=scalars32[1].value,
            feed_calls=scalars32[2].value,
            fetch_calls=scalars32[3].value,
            commit_state=scalars32[4].value,
            kv_import_checksum=scalars32[5].value & 0xFFFFFFFF,
            wall_us=scalars64[0].value,
            native_cpu_us=scalars64[1].value,
            declared_input_bytes=scalars64[2].value,
            declared_output_bytes=scalars64[3].value,
        )

    # -- timing ------------------------------------------------------------------
    def enable_kernel_timing(self, on: bool = True) -> None:
        if self.lib.resident_epoch_kernel_timing(self.handle, 1 if on else 0) != 0:
            raise RuntimeError("kernel timing toggle failed")

    def time_ops(self, begin: int, end: int, iters: int = 20) -> float:
        """Mean ms of the decoder-step launch range [begin, end) (eager, HIP events)."""
        out = ctypes.c_float(0.0)
        rc = self.lib.resident_epoch_time_ops(self.handle, begin, end, iters, ctypes.byref(out))
        if rc != 0:
            raise RuntimeError(f"time_ops failed: {rc}")
        return float(out.value)

    LAYER_OPS = ("qkv", "attention", "o_proj", "o_reduce", "gate_up", "down", "down_reduce")

    def time_layer_op(self, which: str, passes: int = 2) -> float:
        """Mean ms of one layer op launched for every layer in turn, back to
        back (resident_epoch_time_layer_op: each launch streams cold weights)."""
        out = ctypes.c_float(0.0)
        rc = self.lib.resident_epoch_time_layer_op(self.handle, self.LAYER_OPS.index(which), passes, ctypes.byref(out))
        if rc != 0:
            raise RuntimeError(f"time_layer_op failed: {rc}")
        return float(out.value)

    def op_index(self, layer: int, which: str) -> int:
        """Index of one launch in the step's launch list."""
        order = ("qkv", "attention", "o_proj", "o_reduce", "gate_up", "down", "down_reduce")
        if which == "embed":
            return 0
        if which == "lm_head":
            return self.info("step_ops") - 1
        return 1 + self.info("ops_per_layer") * layer + order.index(which)

    def timed_launch_ms(self) -> list[float]:
        """Durations (ms) of the timed launches since the last read (the
        gate/up projection of the timing layer in each epoch's last step):
        one per completed epoch while timing is enabled."""
        n = 4096
        buf = (ctypes.c_float * n)()
        got = self.lib.resident_epoch_read_kernel_timing(self.handle, buf, n)
        if got < 0:
            raise RuntimeError(f"kernel timing unavailable (code {got})")
        return [float(buf[i]) for i in range(got)]

    gateup_times_ms = timed_launch_ms


def default_workdir_env() -> str | None:
    return os.getenv("CRUISE_ENGINE_WORKDIR")


def write_weight_bundle(directory: str | Path, weights: dict[str, Any], inv_freq: Any | None = None) -> Path:
    """Write a weight bundle the engine loads with "weights.source" =
    "bundle": one raw little-endian file per tensor, named as the reference's
    bundle (materialize_runtime_weights.py:53-80), plus the optional fp32
    RoPE table ``inv_freq`` (materialize_runtime_weights.py:341-353)."""
    out = Path(directory)
    out.mkdir(parents=True, exist_ok=True)
    items = dict(weights)
    if inv_freq is not None:
        items["inv_freq"] = inv_freq
    for name, value in items.items():
        if hasattr(value, "detach"):
            value = value.detach().to("cpu").contiguous()
            import torch

            raw = value.view(-1).view(torch.uint8).numpy().tobytes()
        else:
            raw = np.ascontiguousarray(value).tobytes()
        (out / name).write_bytes(raw)
    return out
