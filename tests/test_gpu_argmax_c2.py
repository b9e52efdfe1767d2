"""GPU parity of ArgmaxFinite (controller/g4c_b4_resident_epoch.cpp:99-119)
on one Qwen2.5-7B layer in bf16 (152,064-entry vocabulary, many LM-head
workgroups): the emitted token is the first index of the maximum of the
logits the device's step left behind; exact ties planted by identical
LM-head rows (within a row pair, across workgroups, three-way) go to the
lowest index; a NaN LM-head row gives status 209; and the same K=8 epoch
twice from one resident state gives the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cruise_amd.runtime import pack_feed, tiling_bytes
from oracle.weights import generate_weights
from oracle.workloads import C2, random_tables
from parity import engine_restore, engine_snapshot, first_max, make_runtime, oracle_controller, oracle_restore, oracle_snapshot
from test_gpu_controller_edges import STATUS_NON_FINITE, control_of, prefilled, run_both

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def c2():
    dev = generate_weights(C2.dims, C2.seed, device="cuda")
    cpu = {k: v.cpu() for k, v in dev.items()}
    rt = make_runtime(C2, dev)
    torch.cuda.synchronize()
    yield rt, dev, cpu
    rt.close()


def device_logits(rt, W):
    out = torch.zeros(W.geometry.batch, W.dims.vocab, dtype=torch.float32)
    rt.read_state("logits", out)
    return out.numpy()


def test_argmax_is_first_max_of_device_logits(c2):
    rt, dev, cpu = c2
    W = C2
    B = W.geometry.batch
    rng = np.random.default_rng(8804)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    ctl, rows = prefilled(rt, cpu, W, 8804, table)
    for epoch in range(4):
        hist, ctrl = run_both(rt, ctl, W, rows, 1, [W.eos] * B)
        assert ctrl[3] == 0
        logits = device_logits(rt, W)
        assert np.isfinite(logits).all()
        for r in range(B):
            assert hist[0, r] == first_max(logits[r]), (epoch, r)
        rows.advance(hist, ctrl)


# (lowest, others...): rows of the LM head made identical; the step must emit
# the lowest index.  Same row pair; two workgroups far apart; three-way.
TIE_CASES = [(2 * 777, 2 * 777 + 1), (70001, 150001), (5000, 60000, 150000)]


@pytest.mark.parametrize("tie", TIE_CASES, ids=["row-pair", "workgroups", "three-way"])
def test_planted_tie_goes_to_lowest_index(c2, tie):
    rt, dev, cpu = c2
    W = C2
    B = W.geometry.batch
    rng = np.random.default_rng(8805)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    ctl, rows = prefilled(rt, cpu, W, 8805, table)
    snap = engine_snapshot(rt, torch.bfloat16)
    tok, pos, lens, slots, act = rows.feed_parts()
    feed = pack_feed(tok, pos, lens, slots, act, table, tiling_bytes(), control_of(B, 1, [W.eos] * B, rows.gens))
    rt.proc(feed)
    k0 = first_max(device_logits(rt, W)[0])
    assert k0 not in tie
    lm = dev["lm_head"].clone()
    for i in tie:
        lm[i] = lm[k0] * 4  # a power of two: bf16-exact, every logit scales exactly
    rt.write_state("lm_head", lm)
    try:
        engine_restore(rt, snap)
        hist, ctrl = rt.proc(feed)
        logits = device_logits(rt, W)
    finally:
        rt.write_state("lm_head", dev["lm_head"])
    assert ctrl[3] == 0
    vals = [logits[0, i] for i in tie]
    assert all(v == vals[0] for v in vals) and vals[0] == logits[0].max(), vals
    assert hist[0, 0] == min(tie)
    for r in range(B):
        assert hist[0, r] == first_max(logits[r]), r


def test_nan_logits_fall_back_209(c2):
    rt, dev, cpu = c2
    W = C2
    B = W.geometry.batch
    rng = np.random.default_rng(8806)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    ctl, rows = prefilled(rt, cpu, W, 8806, table)
    lm = dev["lm_head"].clone()
    lm[99999] = float("nan")
    bad = dict(cpu)
    bad["lm_head"] = lm.cpu()
    _, ctl_bad = oracle_controller(W, bad)
    oracle_restore(ctl_bad, oracle_snapshot(ctl))
    rows_before = rt.resident_rows().copy()
    rt.write_state("lm_head", lm)
    try:
        hist, ctrl = run_both(rt, ctl_bad, W, rows, 4, [W.eos] * B)
    finally:
        rt.write_state("lm_head", dev["lm_head"])
    assert ctrl[3] == STATUS_NON_FINITE and ctrl[4] == 1 and (hist == -1).all()
    np.testing.assert_array_equal(rt.resident_rows(), rows_before)


def test_epoch_replay_is_bit_identical(c2):
    """Two K=8 epochs from the same resident state: identical history,
    control record and caches, bit for bit."""
    rt, dev, cpu = c2
    W = C2
    B = W.geometry.batch
    rng = np.random.default_rng(8807)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    ctl, rows = prefilled(rt, cpu, W, 8807, table)
    snap = engine_snapshot(rt, torch.bfloat16)
    tok, pos, lens, slots, act = rows.feed_parts()
    feed = pack_feed(tok, pos, lens, slots, act, table, tiling_bytes(), control_of(B, 8, [W.eos] * B, rows.gens))
    runs = []
    for _ in range(2):
        engine_restore(rt, snap)
        hist, ctrl = rt.proc(feed)
        k, v, res = engine_snapshot(rt, torch.bfloat16)
        runs.append((hist, ctrl, k.cpu(), v.cpu(), res))
    (h1, c1_, k1, v1, r1), (h2, c2_, k2, v2, r2) = runs
    assert c1_[3] == 0 and c1_[4] == 8
    np.testing.assert_array_equal(h1, h2)
    np.testing.assert_array_equal(c1_, c2_)
    np.testing.assert_array_equal(r1, r2)
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
