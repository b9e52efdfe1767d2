"""GPU parity of the controller branches an ordinary epoch does not reach
(controller/g4c_b4_resident_epoch.cpp, "CTRL"):

* device-side EOS (CTRL:577-580): an epoch is run once, then re-run from the
  same resident state with each row's EOS set to a token that row emitted, so
  rows leave the loop at chosen steps -- some rows, and every row before the
  last step of a K=8 epoch (the loop's no-active-row exit, CTRL:488, which on
  the device turns the captured graph's remaining launches into early exits);
* non-finite logits (a +Inf LM-head row) -> status 209 (the NaN case and
  the argmax tie rule run on the 7B vocabulary in test_gpu_argmax_c2.py);
* AlreadyFinished (5) and Empty (4) rows beside active ones.

History and control record are compared bit for bit with the oracle
controller (teacher-forced where the top-2 margin is not decisive), resident
rows exactly, caches at the model tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cruise_amd.runtime import pack_feed, tiling_bytes
from oracle.controller import EpochFeed, control_input_elements
from oracle.weights import generate_weights
from oracle.workloads import C1, identity_table, prompts, slot_of
from parity import (
    TeacherForcing,
    assert_close_rel,
    engine_restore,
    engine_snapshot,
    make_runtime,
    oracle_controller,
    oracle_restore,
    oracle_snapshot,
    rel_tol,
)

pytestmark = pytest.mark.gpu

STATUS_NON_FINITE = 209
FINISH_EOS, FINISH_MAX, FINISH_FALLBACK, FINISH_EMPTY, FINISH_ALREADY = 1, 2, 3, 4, 5


def control_of(B, K, eos, gens):
    c = np.zeros(control_input_elements(B), dtype=np.int32)
    c[0] = K
    c[1 : 1 + B] = eos
    c[3 + B : 3 + 2 * B] = gens
    return c


class Rows:
    """Host view of B rows continuing their generations."""

    def __init__(self, W, table, ps, gens):
        self.W = W
        self.table = table
        self.tokens = np.array([p[-1] for p in ps], dtype=np.int64)
        self.positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
        self.gens = np.asarray(gens, dtype=np.int32)

    def feed_parts(self, active=None):
        B, bs = self.W.geometry.batch, self.W.geometry.block_size
        active = np.ones(B, dtype=np.int32) if active is None else np.asarray(active, dtype=np.int32)
        lengths = (self.positions + 1).astype(np.int32)
        slots = np.array([slot_of(self.table, r, int(self.positions[r]), bs) for r in range(B)], dtype=np.int32)
        return self.tokens.copy(), self.positions.copy(), lengths, slots, active

    def advance(self, hist, ctrl):
        B = self.W.geometry.batch
        executed = ctrl[6 + 2 * B : 6 + 3 * B]
        for r in range(B):
            if executed[r]:
                self.tokens[r] = hist[executed[r] - 1, r]
                self.positions[r] += executed[r]


def run_both(rt, ctl, W, rows, K, eos, *, compare=True):
    """One epoch on the device and in the oracle from their current states."""
    B = W.geometry.batch
    tok, pos, lens, slots, act = rows.feed_parts()
    control = control_of(B, K, eos, rows.gens)
    hist, ctrl = rt.proc(pack_feed(tok, pos, lens, slots, act, rows.table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tok, pos, lens, slots, act, rows.table.reshape(-1), tiling_bytes(), control))
    if compare:
        assert not tf.mismatches, tf.mismatches
        np.testing.assert_array_equal(hist, ref.history)
        np.testing.assert_array_equal(ctrl, ref.control)
    return hist, ctrl


def eos_choice(hist, row, target):
    """(step, token): the latest step <= target whose token is that row's first
    occurrence of it, so an EOS set to the token ends the row exactly there."""
    col = [int(t) for t in hist[:, row]]
    best = 0
    for j in range(min(target, len(col) - 1) + 1):
        if col[j] >= 0 and col[j] not in col[:j]:
            best = j
    return best, col[best]


def check_resident(rt, ctl, W, what):
    rows = rt.resident_rows()
    np.testing.assert_array_equal(rows[0], ctl.resident_generation, err_msg=what)
    np.testing.assert_array_equal(rows[1], ctl.resident_token, err_msg=what)
    np.testing.assert_array_equal(rows[2], ctl.resident_position, err_msg=what)
    np.testing.assert_array_equal(rows[3], ctl.resident_length, err_msg=what)
    dt = W.dims.torch_dtype
    k = torch.zeros(ctl.resident_key.numel(), dtype=dt)
    v = torch.zeros_like(k)
    rt.read_state("key_cache", k)
    rt.read_state("value_cache", v)
    assert_close_rel(k.view_as(ctl.resident_key), ctl.resident_key, rel_tol(W.dims), f"{what}: resident keys")
    assert_close_rel(v.view_as(ctl.resident_value), ctl.resident_value, rel_tol(W.dims), f"{what}: resident values")


@pytest.fixture(scope="module")
def c1():
    weights = generate_weights(C1.dims, C1.seed)
    rt = make_runtime(C1, weights)
    yield rt, weights
    rt.close()


def prefilled(rt, weights, W, seed, table):
    """Fresh zero state, 2-5 token prompts prefilled on both sides."""
    B = W.geometry.batch
    _, ctl = oracle_controller(W, weights)
    dt = W.dims.torch_dtype
    zeros = torch.zeros(rt.cache_bytes // torch.tensor([], dtype=dt).element_size(), dtype=dt, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    rng = np.random.default_rng(seed)
    ps = prompts(rng, B, W.dims.vocab)
    gens = np.arange(1, B + 1, dtype=np.int32) + 100
    for r in range(B):
        rt.prefill(r, int(gens[r]), ps[r], table[r])
        ctl.prefill_row(r, int(gens[r]), ps[r], table[r])
    return ctl, Rows(W, table, ps, gens)


@pytest.mark.parametrize("targets,case", [([1, 3, 99, 6], "some-rows"), ([0, 2, 1, 3], "every-row")])
def test_forced_eos(c1, targets, case):
    rt, weights = c1
    W = C1
    B = W.geometry.batch
    table = identity_table(B, W.geometry.blocks_per_row)
    ctl, rows = prefilled(rt, weights, W, 8801, table)
    snap_gpu, snap_ctl = engine_snapshot(rt, torch.float32), oracle_snapshot(ctl)
    base_hist, _ = run_both(rt, ctl, W, rows, 8, [W.eos] * B)
    assert (base_hist != W.eos).all()
    eos = [W.eos] * B
    stop = [None] * B
    for r in range(B):
        if targets[r] < 8:
            stop[r], eos[r] = eos_choice(base_hist, r, targets[r])
    print(f"[eos] {case}: rows stop at steps {stop}, eos {eos}", flush=True)
    engine_restore(rt, snap_gpu)
    oracle_restore(ctl, snap_ctl)
    hist, ctrl = run_both(rt, ctl, W, rows, 8, eos)
    executed = ctrl[6 + 2 * B : 6 + 3 * B]
    reasons = ctrl[6 + 3 * B : 6 + 4 * B]
    for r in range(B):
        if stop[r] is None:
            assert executed[r] == 8 and reasons[r] == FINISH_MAX
        else:
            assert executed[r] == stop[r] + 1 and reasons[r] == FINISH_EOS, (r, executed, reasons)
            assert hist[stop[r], r] == eos[r] and (hist[stop[r] + 1 :, r] == -1).all()
    # the same tokens as the run without EOS up to each row's stop
    for r in range(B):
        n = executed[r]
        np.testing.assert_array_equal(hist[:n, r], base_hist[:n, r])
    assert ctrl[4] == max(executed)  # model calls
    if case == "every-row":
        assert ctrl[4] < 8 and ctrl[6 + 4 * B + 1] == 0  # the loop left early, no row active
    check_resident(rt, ctl, W, case)


def test_already_finished_and_empty_rows(c1):
    """finished / active / empty / active (b4_eager_test.py:110-120) in an epoch."""
    rt, weights = c1
    W = C1
    B = W.geometry.batch
    table = identity_table(B, W.geometry.blocks_per_row)
    ctl, rows = prefilled(rt, weights, W, 8802, table)
    tok, pos, lens, slots, _ = rows.feed_parts()
    act = np.array([0, 1, 0, 1], dtype=np.int32)
    gens = rows.gens.copy()
    # row 2 is empty: position 0, length 0, generation 0, slot of position 0
    pos[2], lens[2], gens[2] = 0, 0, 0
    slots[2] = slot_of(table, 2, 0, W.geometry.block_size)
    control = control_of(B, 4, [W.eos] * B, gens)
    hist, ctrl = rt.proc(pack_feed(tok, pos, lens, slots, act, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tok, pos, lens, slots, act, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    reasons = ctrl[6 + 3 * B : 6 + 4 * B]
    assert ctrl[3] == 0 and list(reasons) == [FINISH_ALREADY, FINISH_MAX, FINISH_EMPTY, FINISH_MAX]
    assert list(ctrl[6 + 4 * B + 2 :]) == [0, int(gens[1]), 0, int(gens[3])]  # generations acknowledged
    assert (hist[:, 0] == -1).all() and (hist[:, 2] == -1).all()
    check_resident(rt, ctl, W, "finished/empty")


def test_infinite_logits_fall_back_209(c1):
    rt, weights = c1
    W = C1
    B = W.geometry.batch
    table = identity_table(B, W.geometry.blocks_per_row)
    bad = dict(weights)
    lm = weights["lm_head"].clone()
    lm[1234] = float("inf")
    bad["lm_head"] = lm
    ctl, rows = prefilled(rt, weights, W, 8803, table)
    _, ctl_bad = oracle_controller(W, bad)
    oracle_restore(ctl_bad, oracle_snapshot(ctl))
    rows_before = rt.resident_rows().copy()
    rt.write_state("lm_head", lm)
    try:
        hist, ctrl = run_both(rt, ctl_bad, W, rows, 2, [W.eos] * B)
    finally:
        rt.write_state("lm_head", weights["lm_head"])
    assert ctrl[3] == STATUS_NON_FINITE and ctrl[4] == 1
    assert (hist == -1).all() and list(ctrl[6 + 3 * B : 6 + 4 * B]) == [FINISH_FALLBACK] * B
    np.testing.assert_array_equal(rt.resident_rows(), rows_before)  # a fallback saves no resident row
