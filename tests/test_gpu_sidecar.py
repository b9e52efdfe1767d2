"""GPU parity through the sidecar: resident_epoch_server (a child process
holding the engine of the HIP library) driven over its socket by the
Python client and the worker backend, as the reference's worker drives its
sidecar (sidecar_backend.py:67-462, backend.py:90-208).

Tiny fp32 model from a weight bundle in /dev/shm.  Epochs are checked
against the oracle controller fed what the bridge feeds (identity block
table, BRIDGE:524-569): new generations, a continuation, a host-snapshot
KV import whose device checksum must equal the snapshot's, and a device-IPC
import of KV blocks that never leave the GPU.
"""
from __future__ import annotations

import os
import shutil
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch

from cruise_amd.backend import ResidentEpochBackend
from cruise_amd.contract import CONTRACT_VERSION, EpochCommitState, ResidentEpochPlan, ResidentEpochRequest, get_result
from cruise_amd.kv_transfer import KVGeometry, ResidentKVSnapshot, kv_payload_checksum
from cruise_amd.runtime import WeightSpec, tiling_bytes, write_weight_bundle
from cruise_amd.sidecar_backend import SidecarDataFlowEngine
from oracle.controller import IMPORT_GRAPH_FLAG, EpochFeed, control_input_elements
from oracle.decoder import inv_freq
from oracle.weights import generate_weights
from oracle.workloads import C1, identity_table, slot_of
from parity import TeacherForcing, engine_config, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C1
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
GEOMETRY = KVGeometry(W.dims.num_layers, B, BS, W.dims.num_kv_heads, W.dims.head_dim, 4)


@pytest.fixture(scope="module")
def weights():
    return generate_weights(W.dims, W.seed)


@pytest.fixture(scope="module")
def sidecar(weights):
    shm = Path(tempfile.mkdtemp(prefix="cruise-sidecar-gpu-", dir="/dev/shm"))
    files = Path(tempfile.mkdtemp(prefix="cruise-sidecar-cfg-"))
    write_weight_bundle(shm, weights, inv_freq=inv_freq(W.dims).contiguous())
    (files / "graph_config.json").write_text(engine_config(W, weights=WeightSpec("bundle")).to_json())
    (files / "tiling.bin").write_bytes(tiling_bytes())
    (files / "model.air").write_bytes(b"")
    (files / "func.json").write_text("{}")
    env = {
        "VLLM_ASCEND_RESIDENT_EPOCH_AIR": files / "model.air",
        "VLLM_ASCEND_RESIDENT_EPOCH_GRAPH_CONFIG": files / "graph_config.json",
        "VLLM_ASCEND_RESIDENT_EPOCH_FUNC_CONFIG": files / "func.json",
        "VLLM_ASCEND_RESIDENT_EPOCH_TILING": files / "tiling.bin",
        "VLLM_ASCEND_RESIDENT_EPOCH_EXTERNAL_WEIGHTS": shm,
        "VLLM_ASCEND_RESIDENT_EPOCH_SOCKET": shm / "epoch.sock",
        "VLLM_ASCEND_RESIDENT_EPOCH_STARTUP_TIMEOUT": "300",
    }
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update({k: str(v) for k, v in env.items()})
    print("sidecar: starting resident_epoch_server", flush=True)
    eng = SidecarDataFlowEngine()
    eng.warmup_token = 11690 % W.dims.vocab
    eng.warmup_eos = W.eos
    try:
        yield eng
    finally:
        eng.close()
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        shutil.rmtree(shm, ignore_errors=True)
        shutil.rmtree(files, ignore_errors=True)


@pytest.fixture(scope="module")
def oracle(weights):
    _, ctl = oracle_controller(W, weights)
    return ctl


def request(row, gen, token, pos, *, owner="host", imp=False):
    return ResidentEpochRequest(f"req-{gen}", row, gen, token, pos, pos + 1, W.eos, (row,), (BPR * row, BPR * row + 1),
                                state_owner=owner, kv_import_required=imp)


def plan_of(reqs, steps):
    mask = [0] * B
    for r in reqs:
        mask[r.row] = 1
    return ResidentEpochPlan(CONTRACT_VERSION, B, steps, W.geometry.window, tuple(reqs), tuple(mask))


def oracle_epoch(ctl, plan, history, payload=None, mask=0):
    """The oracle controller fed the bridge's feed for this plan."""
    table = identity_table(B, BPR)
    tokens = np.zeros(B, dtype=np.int64)
    positions = np.zeros(B, dtype=np.int64)
    lengths = np.zeros(B, dtype=np.int32)
    active = np.zeros(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = plan.max_steps
    control[1 : 1 + B] = W.eos
    for r in plan.requests:
        tokens[r.row], positions[r.row], lengths[r.row], active[r.row] = r.token_id, r.position, r.sequence_length, 1
        control[1 + r.row] = r.eos_token_id
        control[3 + B + r.row] = r.generation
    if payload is not None:
        control[2 + B] = IMPORT_GRAPH_FLAG | mask
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    ctl.token_override = TeacherForcing(history, rel_tol(W.dims))
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control,
                             import_payload=payload))
    assert not ctl.token_override.mismatches, ctl.token_override.mismatches
    return ref


def history_of(out, plan):
    hist = np.full((8, B), -1, dtype=np.int64)
    for r in plan.requests:
        toks = out.sampled_token_ids[out.req_id_to_index[r.req_id]]
        hist[: len(toks), r.row] = toks
    return hist


def check_against_oracle(out, plan, ref):
    result = get_result(out)
    executed = ref.control[6 + 2 * B : 6 + 3 * B]
    for r in plan.requests:
        n = int(executed[r.row])
        assert result.computed_steps[r.req_id] == n
        assert out.sampled_token_ids[out.req_id_to_index[r.req_id]] == [int(t) for t in ref.history[:n, r.row]]
    assert result.model_calls == int(ref.control[4])


def test_warm_up_through_the_server(sidecar):
    backend = ResidentEpochBackend(sidecar)
    w = backend.warm_up()
    assert w.commit_state == EpochCommitState.COMMITTED and w.model_calls == 1
    assert w.declared_input_bytes == 260 and w.declared_output_bytes == 368


def test_epochs_match_the_oracle(sidecar, oracle):
    backend = ResidentEpochBackend(sidecar)
    plan = plan_of([request(r, r + 1, 11 * (r + 1), 0) for r in range(B)], steps=4)
    print("sidecar: new generations K=4", flush=True)
    out = backend.execute(plan)
    result = get_result(out)
    assert result.route == "device" and result.feed_calls == 1 and result.fetch_calls == 1
    ref = oracle_epoch(oracle, plan, history_of(out, plan))
    check_against_oracle(out, plan, ref)

    # the same generations continue from where the epoch stopped (device-owned rows)
    reqs = []
    for r in plan.requests:
        toks = out.sampled_token_ids[out.req_id_to_index[r.req_id]]
        if toks and toks[-1] != W.eos and len(toks) == plan.max_steps:
            reqs.append(request(r.row, r.generation, toks[-1], r.position + len(toks), owner="device"))
    assert reqs, "every row ended at EOS"
    plan2 = plan_of(reqs, steps=2)
    print("sidecar: continuation K=2", flush=True)
    out2 = backend.execute(plan2)
    ref2 = oracle_epoch(oracle, plan2, history_of(out2, plan2))
    check_against_oracle(out2, plan2, ref2)


def test_snapshot_import_through_the_server(sidecar, oracle):
    backend = ResidentEpochBackend(sidecar)
    g = torch.Generator().manual_seed(77)
    payload = (torch.randn(GEOMETRY.payload_bytes // 4, generator=g) * 0.25).numpy().astype(np.float32).tobytes()
    mask = 0b1010
    snap = ResidentKVSnapshot(4242, mask, (0, 21, 0, 22), payload, kv_payload_checksum(payload, mask, GEOMETRY), GEOMETRY)
    plan = plan_of([request(1, 21, 35, 3, imp=True), request(3, 22, 36, 5, imp=True)], steps=2)
    print("sidecar: host-snapshot import K=2", flush=True)
    out = backend.execute(plan, snapshot=snap)
    result = get_result(out)
    assert result.kv_imported and result.kv_import_checksum == snap.checksum
    assert not sidecar.transfer_path.exists()
    ref = oracle_epoch(oracle, plan, history_of(out, plan), payload=payload, mask=mask)
    check_against_oracle(out, plan, ref)


def test_device_ipc_import_through_the_server(sidecar, oracle):
    """The KV blocks stay on the GPU: this process holds the stock caches
    (one [blocks, block_size, kv_heads, head] tensor per layer and cache),
    exports their allocations with HIP IPC, and the server's engine maps them
    and gathers the imported rows' blocks device to device."""
    from types import SimpleNamespace

    from cruise_amd.kv_transfer import capture_kv_device_transfer, release_kv_device_exports

    backend = ResidentEpochBackend(sidecar)
    g = torch.Generator().manual_seed(91)
    shape = (W.geometry.physical_blocks, BS, W.dims.num_kv_heads, W.dims.head_dim)
    caches = [tuple((torch.randn(shape, generator=g) * 0.25).cuda() for _ in range(2)) for _ in range(W.dims.num_layers)]
    torch.cuda.synchronize()
    worker = SimpleNamespace(model_runner=SimpleNamespace(kv_caches=caches))
    blocks = {0: 5, 2: 2}
    reqs = [
        ResidentEpochRequest("ipc-0", 0, 31, 40, 4, 5, W.eos, (blocks[0],), (0, 1), kv_import_required=True),
        ResidentEpochRequest("ipc-2", 2, 32, 41, 2, 3, W.eos, (blocks[2],), (4, 5), kv_import_required=True),
    ]
    plan = plan_of(reqs, steps=2)
    transfer = capture_kv_device_transfer(worker, plan)
    assert transfer.geometry == GEOMETRY and transfer.import_mask == 0b0101
    # the payload the host path would have carried, for the checksum and the oracle
    zero = torch.zeros(shape[1:])
    parts = [[caches[l][kv][blocks[r]].cpu() if r in blocks else zero for l in range(W.dims.num_layers) for r in range(B)]
             for kv in range(2)]
    payload = b"".join(torch.stack(p).numpy().astype(np.float32).tobytes() for p in parts)
    print("sidecar: device-IPC import K=2", flush=True)
    out = backend.execute(plan, device_transfer=transfer)
    result = get_result(out)
    assert result.kv_transfer_mode == "device_ipc"
    assert result.declared_input_bytes == 136 + 4088
    assert result.kv_import_checksum == kv_payload_checksum(payload, 0b0101, GEOMETRY)
    ref = oracle_epoch(oracle, plan, history_of(out, plan), payload=payload, mask=0b0101)
    check_against_oracle(out, plan, ref)
    release_kv_device_exports(worker)
    del caches
