"""The scheduler's plans, end to end on the GPU.

The resident-epoch scheduler (cruise_amd.scheduler over the in-memory
vLLM-shaped base scheduler of tests/fake_vllm.py) plans every step.  Its
plans run through the worker backend and the sidecar server, whose engine is
the HIP library holding one Qwen2.5-7B layer (bf16, vocabulary 152,064).
Each epoch is checked against the oracle controller fed the bridge's feed for
the same plan (identity block table, BRIDGE:524-569), teacher-forced by the
GPU's tokens where the top-2 margin is not decisive: sampled tokens,
executed steps, model calls and generations bit for bit.  Then the scheduler
takes the output back (update_from_output), which validates the result
against the plan and advances its accounting.

Two cohorts:

* the reference's (run_multi_epoch_cohort.py:128-278,
  verify_multi_epoch_cohort_result.py:28-63): prompts of the single token
  11690, budgets A 6, B 2, C 2, K at most 2, capacity 8.  The three epochs
  must have the reference's rows, generations, positions and input tokens,
  and B's and C's tokens must equal A's first two (a reused row starts from
  cleared blocks).
* a prefilled one: 2-5 token prompts.  Each prompt is prefilled on the host
  lane -- the oracle decoder stands in for the stock model, writing a stock
  paged KV cache of the base scheduler's blocks -- and enters the device by
  a host-snapshot KV import captured from that cache
  (kv_transfer.capture_kv_snapshot).  B and C are prefilled while A is
  device-owned, so the scheduler isolates the host lane (scheduler.py:102-161).
"""
from __future__ import annotations

import os
import shutil
import tempfile
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from cruise_amd.backend import ModelRunnerOutput, ResidentEpochBackend
from cruise_amd.config import ResidentEpochConfig
from cruise_amd.contract import get_plan, get_result
from cruise_amd.kv_transfer import capture_kv_snapshot
from cruise_amd.runtime import WeightSpec, tiling_bytes, write_weight_bundle
from cruise_amd.scheduler import ResidentEpochSchedulerMixin
from cruise_amd.sidecar_backend import SidecarDataFlowEngine
from fake_vllm import FakeScheduler, Request, greedy_params
from oracle.controller import IMPORT_GRAPH_FLAG, EpochFeed, argmax_finite, control_input_elements
from oracle.decoder import OracleDecoder, PagedGeometry, inv_freq
from oracle.weights import generate_weights
from oracle.workloads import C2, identity_table, slot_of
from parity import TeacherForcing, engine_config, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C2
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
HOST_BLOCKS = 16  # the base scheduler's KV blocks (FakeScheduler default)
WARM_TOKEN = 11690


class Scheduler(ResidentEpochSchedulerMixin, FakeScheduler):
    pass


@pytest.fixture(scope="module")
def weights():
    print("[sched-cohort] generating one-layer 7B weights", flush=True)
    dev = generate_weights(W.dims, W.seed, device="cuda")
    cpu = {k: v.cpu() for k, v in dev.items()}
    del dev
    torch.cuda.empty_cache()
    return cpu


@pytest.fixture(scope="module")
def backend(weights):
    shm = Path(tempfile.mkdtemp(prefix="cruise-sched-gpu-", dir="/dev/shm"))
    files = Path(tempfile.mkdtemp(prefix="cruise-sched-cfg-"))
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
    print("[sched-cohort] starting resident_epoch_server", flush=True)
    eng = SidecarDataFlowEngine()
    try:
        yield ResidentEpochBackend(eng)
    finally:
        eng.close()
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        shutil.rmtree(shm, ignore_errors=True)
        shutil.rmtree(files, ignore_errors=True)


class HostLane:
    """The stock model of the host lane: the oracle decoder over a stock
    paged cache of the base scheduler's blocks ([blocks, block_size,
    kv_heads, head] per layer)."""

    def __init__(self, weights, capacity):
        self.model = OracleDecoder(W.dims, PagedGeometry(B, HOST_BLOCKS, BS, 1, capacity), weights)
        shape = self.model.cache_shape()
        self.key = torch.zeros(shape, dtype=W.dims.torch_dtype)
        self.value = torch.zeros(shape, dtype=W.dims.torch_dtype)
        self.worker = SimpleNamespace(model_runner=SimpleNamespace(
            kv_caches=[(self.key[l], self.value[l]) for l in range(W.dims.num_layers)]))

    def prefill(self, prompt: list[int], block: int) -> int:
        """Run the prompt at positions 0..L-1 into ``block`` and return the
        greedy first token."""
        table = np.zeros((B, 1), dtype=np.int32)
        table[0, 0] = block
        logits = None
        for p, token in enumerate(prompt):
            tok = np.zeros((B, 1), dtype=np.int64)
            pos = np.zeros(B, dtype=np.int64)
            length = np.zeros((B, 1), dtype=np.int32)
            slot = np.full(B, -1, dtype=np.int32)
            act = np.zeros(B, dtype=np.int32)
            tok[0, 0], pos[0], length[0, 0], slot[0], act[0] = token, p, p + 1, block * BS + p, 1
            logits, *_ = self.model.forward(torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length),
                                            torch.from_numpy(table), torch.from_numpy(slot), self.key, self.value,
                                            torch.zeros(72, dtype=torch.uint8), torch.from_numpy(act), inplace=True)
        first = argmax_finite(logits[0, 0].numpy())
        assert first is not None
        return first


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


def run_device_epoch(backend, ctl, plan, snapshot, label):
    out = backend.execute(plan, snapshot=snapshot)
    result = get_result(out)
    assert result.route == "device" and (result.feed_calls, result.fetch_calls) == (1, 1), label
    history = np.full((8, B), -1, dtype=np.int64)
    for r in plan.requests:
        toks = out.sampled_token_ids[out.req_id_to_index[r.req_id]]
        history[: len(toks), r.row] = toks
    ref = oracle_epoch(ctl, plan, history, snapshot.payload if snapshot else None,
                       snapshot.import_mask if snapshot else 0)
    executed = ref.control[6 + 2 * B : 6 + 3 * B]
    for r in plan.requests:
        n = int(executed[r.row])
        assert result.computed_steps[r.req_id] == n, label
        assert out.sampled_token_ids[out.req_id_to_index[r.req_id]] == [int(t) for t in ref.history[:n, r.row]], label
    assert result.model_calls == int(ref.control[4]), label
    assert list(ref.control[6 + 4 * B + 2 : 6 + 5 * B + 2]) == list(result.row_generations), label
    if snapshot is not None:
        assert result.kv_imported and result.kv_import_checksum == snapshot.checksum, label
    return out


def drive(backend, weights, prompts, budgets, config, arrivals):
    """Run the scheduler until every request finished.  ``arrivals`` maps a
    request name to (device epochs that must have run, a request that must
    have finished or None) before it is added.  Returns the device epochs as
    (plan, sampled tokens per request), the requests, the host steps and the
    scheduler's rejection reasons for them."""
    s = Scheduler(max_num_seqs=B, num_blocks=HOST_BLOCKS)
    s._resident_epoch_config = config
    _, ctl = oracle_controller(W, weights)
    host = HostLane(weights, config.logical_capacity)
    reqs = {n: Request(n, list(prompts[n]), greedy_params(budgets[n], eos=W.eos)) for n in prompts}
    pending = dict(arrivals)
    epochs, host_steps, rejections = [], [], []
    for _ in range(64):
        for name, (min_epochs, after) in list(pending.items()):
            if len(epochs) >= min_epochs and (after is None or reqs[after].status.value.startswith("finished")):
                s.add_request(reqs[name])
                del pending[name]
        if not s.running and not s.waiting and not pending:
            break
        out = s.schedule()
        plan = get_plan(out)
        if plan is None:
            # host lane: prefill every scheduled prompt and sample its first token
            rejections.append(s._resident_epoch_last_rejection)
            ids = list(out.num_scheduled_tokens)
            tokens = []
            for rid in ids:
                r = reqs[rid]
                assert out.num_scheduled_tokens[rid] == r.num_prompt_tokens, "only prefill runs on the host here"
                block = s.kv_cache_manager.get_blocks(rid).get_block_ids()[0][0]
                tokens.append([host.prefill(r.prompt_token_ids, block)])
            host_steps.append(tuple(ids))
            print(f"[sched-cohort] host prefill {ids} ({rejections[-1]})", flush=True)
            s.update_from_output(out, ModelRunnerOutput(ids, {r: i for i, r in enumerate(ids)}, tokens))
            continue
        snapshot = capture_kv_snapshot(host.worker, plan) if any(r.kv_import_required for r in plan.requests) else None
        label = f"epoch {len(epochs) + 1} rows {[(r.req_id, r.row, r.generation) for r in plan.requests]} K={plan.max_steps}"
        print(f"[sched-cohort] {label} import={snapshot is not None}", flush=True)
        mro = run_device_epoch(backend, ctl, plan, snapshot, label)
        epochs.append((plan, {rid: mro.sampled_token_ids[i] for rid, i in mro.req_id_to_index.items()}))
        s.update_from_output(out, mro)
    else:
        raise AssertionError("the cohort did not finish")
    for r in reqs.values():
        assert r.num_output_tokens == budgets[r.request_id] or r.output_token_ids[-1] == W.eos
    return epochs, reqs, host_steps, rejections


def test_reference_cohort_through_the_scheduler(backend, weights):
    """verify_multi_epoch_cohort_result.py:29-63 with this model's tokens in
    place of the real checkpoint's."""
    config = ResidentEpochConfig(max_steps=2, logical_capacity=8)
    prompts = {"A": [WARM_TOKEN], "B": [WARM_TOKEN], "C": [WARM_TOKEN]}
    arrivals = {"A": (0, None), "B": (1, None), "C": (1, "B")}
    epochs, reqs, host_steps, _ = drive(backend, weights, prompts, {"A": 6, "B": 2, "C": 2}, config, arrivals)
    assert host_steps == []  # one-token prompts never need the host lane
    a = reqs["A"].output_token_ids
    expected = [
        ((1, 0, 0, 0), (1, 0, 0, 0), {"A": (0, 1, 0, WARM_TOKEN)}, {"A": a[:2]}),
        ((1, 1, 0, 0), (1, 2, 0, 0), {"A": (0, 1, 2, a[1]), "B": (1, 2, 0, WARM_TOKEN)}, {"A": a[2:4], "B": a[:2]}),
        ((1, 1, 0, 0), (1, 3, 0, 0), {"A": (0, 1, 4, a[3]), "C": (1, 3, 0, WARM_TOKEN)}, {"A": a[4:6], "C": a[:2]}),
    ]
    assert len(epochs) == 3
    for (plan, sampled), (mask, gens, rows, tokens) in zip(epochs, expected):
        assert plan.max_steps == 2 and plan.logical_capacity == 8
        assert plan.active_mask == mask and plan.row_generations == gens
        assert {r.req_id: (r.row, r.generation, r.position, r.token_id) for r in plan.requests} == rows
        assert not any(r.kv_import_required for r in plan.requests)
        assert sampled == tokens
    assert reqs["B"].output_token_ids == reqs["C"].output_token_ids == a[:2]
    for r in reqs.values():
        assert r.num_computed_tokens == r.num_tokens - 1  # the last sampled token is never fed back


def test_prefilled_cohort_with_kv_imports(backend, weights):
    rng = np.random.default_rng(W.seed + 40)
    prompts = {n: list(map(int, rng.integers(0, W.dims.vocab, size=L))) for n, L in (("A", 3), ("B", 4), ("C", 2))}
    budgets = {"A": 9, "B": 2, "C": 4}
    config = ResidentEpochConfig(max_steps=4, logical_capacity=16)
    arrivals = {"A": (0, None), "B": (1, None), "C": (1, "B")}
    epochs, reqs, host_steps, rejections = drive(backend, weights, prompts, budgets, config, arrivals)
    # every prompt is prefilled on the host; B's and C's beside a device-owned A
    assert host_steps == [("A",), ("B",), ("C",)]
    assert rejections == ["not-single-token-decode", "host-prefill-admission", "host-prefill-admission"]
    seen = {}
    for plan, _ in epochs:
        for r in plan.requests:
            first = r.req_id not in seen
            seen.setdefault(r.req_id, (r.row, r.generation))
            assert (r.row, r.generation) == seen[r.req_id]
            # the first epoch of a prefilled request imports its KV, later ones find it resident
            assert r.kv_import_required == first and r.state_owner == ("host" if first else "device")
            if first:
                assert r.position == len(prompts[r.req_id])
    assert seen == {"A": (0, 1), "B": (1, 2), "C": (1, 3)}
    assert [p.max_steps for p, _ in epochs[:3]] == [4, 1, 2]
