"""Device-IPC KV import at the reference's geometry, through the sidecar.

The reference's worker exports its stock KV allocations and the sidecar's
engine maps them and copies each imported row's block of every layer on the
device (native/resident_epoch_bridge.cpp:156-273,
src/vllm_ascend_resident_epoch/kv_transfer.py:266-352).  Here, at the
Qwen2.5-7B geometry (28 layers, 4 KV heads x 128, blocks of 128 positions,
bf16):

* an exporter child process (tests/ipc_exporter.py) holds 28 x (K, V)
  stock caches, each its own allocation (56 IPC handles, every key slot of
  the 4,088-byte record used, each allocation far below 2 GiB), and builds
  the record with ``capture_kv_device_transfer``;
* the sidecar server runs the full 7B engine (synthetic weights generated
  on the device) and imports two rows (mask 0b1010) from the exporter's
  allocations, then runs a K=2 epoch;
* the device checksum equals zlib.adler32 over the same blocks in the
  reference's order (K then V, layer-major, rows ascending), computed here
  from the host-path payload the exporter wrote;
* the epoch's tokens, executed counts and model calls equal the oracle
  controller's, fed that payload as an import (teacher-forced where the
  top-2 margin is within the bf16 tolerance).
"""
from __future__ import annotations

import json
import os
import shutil
import subprocess
import sys
import tempfile
import zlib
from pathlib import Path

import numpy as np
import pytest
import torch

from cruise_amd.backend import ResidentEpochBackend
from cruise_amd.contract import CONTRACT_VERSION, ResidentEpochPlan, ResidentEpochRequest, get_result
from cruise_amd.kv_transfer import IPC_KEY_BYTES, IPC_METADATA_BYTES, DeviceKVTransfer, KVGeometry
from cruise_amd.runtime import ResidentEpochRuntime, WeightSpec, tiling_bytes
from cruise_amd.sidecar_backend import SidecarDataFlowEngine
from oracle.controller import IMPORT_GRAPH_FLAG, EpochFeed, control_input_elements
from oracle.decoder import weight_shapes
from oracle.workloads import C3, identity_table, slot_of
from parity import TeacherForcing, engine_config, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C3
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
KVG = KVGeometry(W.dims.num_layers, B, BS, W.dims.num_kv_heads, W.dims.head_dim, 2)
STOCK_BLOCKS = 96  # 12 MiB per cache: each one its own allocation
IMPORTS = [(1, 41, 37), (3, 42, 90)]  # (row, generation, stock block)
POSITIONS = {1: 45, 3: 101}


@pytest.fixture(scope="module")
def weights_cpu():
    """The synthetic weights the server generates, read back from an engine
    built from the same seed in this process."""
    rt = ResidentEpochRuntime(engine_config(W, weights=WeightSpec("synthetic", W.seed, 0.02)))
    cpu = {}
    for name, shape in weight_shapes(W.dims).items():
        t = torch.empty(shape, dtype=torch.bfloat16)
        rt.read_state(name, t)
        cpu[name] = t
    rt.close()
    torch.cuda.empty_cache()
    return cpu


def start_sidecar(shm: Path, files: Path) -> SidecarDataFlowEngine:
    (files / "graph_config.json").write_text(engine_config(W, weights=WeightSpec("synthetic", W.seed, 0.02)).to_json())
    (files / "tiling.bin").write_bytes(tiling_bytes())
    (files / "model.air").write_bytes(b"")
    (files / "func.json").write_text("{}")
    os.environ.update({
        "VLLM_ASCEND_RESIDENT_EPOCH_AIR": str(files / "model.air"),
        "VLLM_ASCEND_RESIDENT_EPOCH_GRAPH_CONFIG": str(files / "graph_config.json"),
        "VLLM_ASCEND_RESIDENT_EPOCH_FUNC_CONFIG": str(files / "func.json"),
        "VLLM_ASCEND_RESIDENT_EPOCH_TILING": str(files / "tiling.bin"),
        "VLLM_ASCEND_RESIDENT_EPOCH_EXTERNAL_WEIGHTS": str(shm),
        "VLLM_ASCEND_RESIDENT_EPOCH_SOCKET": str(shm / "epoch.sock"),
        "VLLM_ASCEND_RESIDENT_EPOCH_STARTUP_TIMEOUT": "300",
    })
    return SidecarDataFlowEngine()


def reference_checksum(payload: bytes, rows: list[int]) -> int:
    """kv_transfer.py:159-174 restated: zlib.adler32 chained over each
    selected block, K cache first, then V, layer-major, rows ascending."""
    view = memoryview(payload)
    value = 1
    for half in range(2):
        for layer in range(KVG.layers):
            for row in rows:
                start = half * KVG.cache_bytes + (layer * B + row) * KVG.block_bytes
                value = zlib.adler32(view[start : start + KVG.block_bytes], value)
    return value & 0xFFFFFFFF


def oracle_import_epoch(ctl, plan: ResidentEpochPlan, history: np.ndarray, payload: bytes, mask: int):
    """The oracle controller fed what the bridge feeds for an import epoch."""
    table = identity_table(B, BPR)
    tokens = np.zeros(B, dtype=np.int64)
    positions = np.zeros(B, dtype=np.int64)
    lengths = np.zeros(B, dtype=np.int32)
    active = np.zeros(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = plan.max_steps
    control[1 : 1 + B] = W.eos
    control[2 + B] = IMPORT_GRAPH_FLAG | mask
    for r in plan.requests:
        tokens[r.row], positions[r.row], lengths[r.row], active[r.row] = r.token_id, r.position, r.sequence_length, 1
        control[3 + B + r.row] = r.generation
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    ctl.token_override = TeacherForcing(history, rel_tol(W.dims))
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control,
                             import_payload=payload))
    assert not ctl.token_override.mismatches, ctl.token_override.mismatches
    return ref


def test_device_ipc_import_at_qwen7b_geometry_through_the_server(weights_cpu):
    shm = Path(tempfile.mkdtemp(prefix="cruise-ipc7b-", dir="/dev/shm"))
    files = Path(tempfile.mkdtemp(prefix="cruise-ipc7b-cfg-"))
    payload_path = shm / "payload.bin"
    saved = {k: v for k, v in os.environ.items() if k.startswith("VLLM_ASCEND_RESIDENT_EPOCH_")}
    exporter = sidecar = None
    try:
        args = {"layers": KVG.layers, "blocks": STOCK_BLOCKS, "block_size": BS, "kv_heads": KVG.kv_heads,
                "head_dim": KVG.head_size, "batch": B, "seed": 8080, "imports": IMPORTS,
                "payload_path": str(payload_path)}
        print("ipc7b: starting the exporter", flush=True)
        exporter = subprocess.Popen([sys.executable, "-u", str(Path(__file__).with_name("ipc_exporter.py")),
                                     json.dumps(args)], stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True)
        line = exporter.stdout.readline()
        assert line, f"the exporter ended without a record (status {exporter.poll()})"
        rec = json.loads(line)
        transfer = DeviceKVTransfer(rec["transfer_id"], rec["import_mask"], tuple(rec["row_generations"]),
                                    tuple(rec["block_ids"]), rec["source_bytes"], tuple(rec["source_offsets"]),
                                    tuple(bytes.fromhex(k) for k in rec["keys"]), KVG)
        assert rec["allocations"] == 2 * KVG.layers == len(set(transfer.keys)) == 56
        assert transfer.source_bytes < 2 << 30 and set(transfer.source_offsets) == {0}
        wire = transfer.wire_bytes()
        assert len(wire) == IPC_METADATA_BYTES == 4088 and all(any(k) for k in transfer.keys)
        assert len(transfer.keys[0]) == IPC_KEY_BYTES
        payload = payload_path.read_bytes()
        assert len(payload) == KVG.payload_bytes == 29_360_128

        print("ipc7b: starting the sidecar (Qwen2.5-7B, synthetic weights)", flush=True)
        sidecar = start_sidecar(shm, files)
        backend = ResidentEpochBackend(sidecar)
        reqs = [ResidentEpochRequest(f"ipc-{row}", row, gen, 1000 + row, POSITIONS[row], POSITIONS[row] + 1, W.eos,
                                     (block,), (BPR * row, BPR * row + 1), kv_import_required=True)
                for row, gen, block in IMPORTS]
        mask = sum(1 << row for row, _, _ in IMPORTS)
        plan = ResidentEpochPlan(CONTRACT_VERSION, B, 2, W.geometry.window, tuple(reqs),
                                 tuple(int(r in POSITIONS) for r in range(B)))
        print("ipc7b: device-IPC import, K=2", flush=True)
        out = backend.execute(plan, device_transfer=transfer)
        result = get_result(out)
        assert result.kv_transfer_mode == "device_ipc" and result.kv_imported
        assert result.declared_input_bytes == 136 + 4088
        assert result.kv_import_checksum == reference_checksum(payload, sorted(POSITIONS))

        print("ipc7b: oracle epoch", flush=True)
        history = np.full((8, B), -1, dtype=np.int64)
        for r in reqs:
            toks = out.sampled_token_ids[out.req_id_to_index[r.req_id]]
            history[: len(toks), r.row] = toks
        _, ctl = oracle_controller(W, weights_cpu)
        ref = oracle_import_epoch(ctl, plan, history, payload, mask)
        executed = ref.control[6 + 2 * B : 6 + 3 * B]
        for r in reqs:
            n = int(executed[r.row])
            assert n == 2 and result.computed_steps[r.req_id] == n
            assert out.sampled_token_ids[out.req_id_to_index[r.req_id]] == [int(t) for t in ref.history[:n, r.row]]
        assert result.model_calls == int(ref.control[4]) == 2
        assert np.uint32(np.int32(ref.control[5])) == result.kv_import_checksum
    finally:
        if sidecar is not None:
            sidecar.close()
        if exporter is not None:
            if exporter.poll() is None:
                exporter.stdin.write("\n")
                exporter.stdin.flush()
            exporter.wait(timeout=60)
        for k in [k for k in os.environ if k.startswith("VLLM_ASCEND_RESIDENT_EPOCH_")]:
            os.environ.pop(k)
        os.environ.update(saved)
        shutil.rmtree(shm, ignore_errors=True)
        shutil.rmtree(files, ignore_errors=True)
