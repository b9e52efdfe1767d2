"""GPU parity on the tiny fp32 model (2 layers, hidden 256, 4/2 heads,
head_dim 64, vocab 4096, block 16 x 2 blocks per row): decoder step, epoch,
fallback codes and the bridge call, each against the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bridge as obridge
from oracle.controller import EpochFeed, control_input_elements
from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C1, prompts, slot_of
from cruise_amd.runtime import pack_feed, tiling_bytes
from parity import TeacherForcing, assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C1
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
CAP = W.geometry.window
FROZEN_TABLE = np.asarray([[1, 0], [3, 2], [5, 4], [7, 6]], dtype=np.int32)  # b4_eager_test.py:79-84


@pytest.fixture(scope="module")
def weights():
    return generate_weights(W.dims, W.seed)


@pytest.fixture(scope="module")
def rt(weights):
    r = make_runtime(W, weights)
    yield r
    r.close()


def b4_cases(rng):
    """The reference's three B=4 cases (b4_eager_test.py:92-120), tokens from the seed."""
    t = rng.integers(0, W.dims.vocab, size=4)
    return [
        ("all-active-heterogeneous", t.copy(), [0, 1, 2, 3], [1, 2, 3, 4], [1, 1, 1, 1]),
        ("two-active-two-empty", np.array([t[0], 0, t[2], 0]), [1, 0, 2, 0], [2, 0, 3, 0], [1, 0, 1, 0]),
        ("finished-active-empty-active", np.array([t[3], t[1], 0, t[2]]), [3, 1, 0, 2], [4, 2, 0, 3], [0, 1, 0, 1]),
    ]


@pytest.mark.parametrize("case_index", [0, 1, 2])
def test_decoder_step_matches_oracle(rt, weights, case_index):
    rng = np.random.default_rng(670100 + case_index)
    name, tok, pos, length, act = b4_cases(rng)[case_index]
    dec, _ = oracle_controller(W, weights)
    shape = dec.cache_shape()
    key, value = seeded_cache(shape, 670100 + case_index, torch.float32)
    slot = np.array([slot_of(FROZEN_TABLE, r, pos[r], BS) for r in range(B)], dtype=np.int32)
    tok64 = np.asarray(tok, dtype=np.int64).reshape(B, 1)
    pos64 = np.asarray(pos, dtype=np.int64)
    len32 = np.asarray(length, dtype=np.int32).reshape(B, 1)
    act32 = np.asarray(act, dtype=np.int32)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok64), torch.from_numpy(pos64), torch.from_numpy(len32), torch.from_numpy(FROZEN_TABLE),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(act32),
    )
    gk = key.clone()
    gv = value.clone()
    logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32)
    nxt = torch.zeros(B, dtype=torch.int64)
    rt.decoder_step(tok64, pos64, len32, gk, slot, act32, FROZEN_TABLE, gv, logits, nxt)
    assert torch.equal(nxt, ref_next), name
    assert_close_rel(logits, ref_logits.reshape(B, -1), rel_tol(W.dims), f"{name} logits")
    # written slots to tolerance, every other slot bit-identical
    flat_ref_k = ref_k.reshape(W.dims.num_layers, -1, W.dims.num_kv_heads, W.dims.head_dim)
    flat_gk = gk.reshape_as(flat_ref_k)
    flat_in = key.reshape_as(flat_ref_k)
    written = [int(slot[r]) for r in range(B) if act[r]]
    mask = torch.ones(flat_in.shape[1], dtype=torch.bool)
    mask[written] = False
    assert torch.equal(flat_gk[:, mask], flat_in[:, mask]), f"{name}: unaddressed key slots changed"
    assert_close_rel(flat_gk[:, written], flat_ref_k[:, written], rel_tol(W.dims), f"{name} written keys")
    flat_ref_v = ref_v.reshape_as(flat_ref_k)
    flat_gv = gv.reshape_as(flat_ref_k)
    assert torch.equal(flat_gv[:, mask], value.reshape_as(flat_ref_k)[:, mask])
    assert_close_rel(flat_gv[:, written], flat_ref_v[:, written], rel_tol(W.dims), f"{name} written values")


def epoch_feed(tokens, positions, lengths, active, table, control):
    slots = [slot_of(table, r, int(positions[r]), BS) for r in range(B)]
    return pack_feed(tokens, positions, lengths, slots, active, table, tiling_bytes(), control)


def test_epoch_matches_oracle_with_prefill(rt, weights):
    """Prompts of 2-5 tokens are prefilled, then two K=2 epochs continue the
    same generations; history, control record, resident rows bit-exact;
    final caches to tolerance."""
    rng = np.random.default_rng(W.seed)
    ps = prompts(rng, B, W.dims.vocab)
    table = FROZEN_TABLE
    dec, ctl = oracle_controller(W, weights)
    # fresh engine state for this test: zero caches and rows
    rt.write_state("key_cache", torch.zeros(rt.cache_bytes // 4, dtype=torch.float32))
    rt.write_state("value_cache", torch.zeros(rt.cache_bytes // 4, dtype=torch.float32))
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    for r in range(B):
        rt.prefill(r, r + 1, ps[r], table[r])
        ctl.prefill_row(r, r + 1, ps[r], table[r])
    rows = rt.resident_rows()
    assert rows[0].tolist() == [1, 2, 3, 4]
    assert rows[2].tolist() == [len(p) - 1 for p in ps]
    tokens = np.array([p[-1] for p in ps], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
    for epoch in range(2):
        lengths = (positions + 1).astype(np.int32)
        active = np.ones(B, dtype=np.int32)
        control = np.zeros(control_input_elements(B), dtype=np.int32)
        control[0] = 2
        control[1 : 1 + B] = W.eos
        control[3 + B : 3 + 2 * B] = np.arange(1, B + 1)
        feed = epoch_feed(tokens, positions, lengths, active, table, control)
        hist, ctrl_out = rt.proc(feed)
        tf = TeacherForcing(hist, rel_tol(W.dims))
        ctl.token_override = tf
        slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
        ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control))
        assert not tf.mismatches, f"epoch {epoch}: decisive token mismatches {tf.mismatches}"
        np.testing.assert_array_equal(hist, ref.history)
        np.testing.assert_array_equal(ctrl_out, ref.control)
        executed = ctrl_out[6 + 2 * B : 6 + 3 * B]
        assert ctrl_out[3] == 0
        for r in range(B):
            if executed[r]:
                tokens[r] = hist[executed[r] - 1, r]
                positions[r] += executed[r]
        rows = rt.resident_rows()
        np.testing.assert_array_equal(rows[0], ctl.resident_generation)
        np.testing.assert_array_equal(rows[1], ctl.resident_token)
        np.testing.assert_array_equal(rows[2], ctl.resident_position)
        np.testing.assert_array_equal(rows[3], ctl.resident_length)
        if np.any(hist[:, :] == W.eos):
            break
    gk = torch.zeros(ctl.resident_key.numel(), dtype=torch.float32)
    rt.read_state("key_cache", gk)
    assert_close_rel(gk.view_as(ctl.resident_key), ctl.resident_key, rel_tol(W.dims), "resident keys")
    gv = torch.zeros_like(gk)
    rt.read_state("value_cache", gv)
    assert_close_rel(gv.view_as(ctl.resident_value), ctl.resident_value, rel_tol(W.dims), "resident values")


FALLBACK_CASES = [
    # (name, mutate(feed dict)) -> expected device status
    ("sampling", lambda f: f["control"].__setitem__(1 + B, 1), 205),
    ("variant", lambda f: f["control"].__setitem__(2 + B, 7), 206),
    ("k-zero", lambda f: f["control"].__setitem__(0, 0), 201),
    ("k-nine", lambda f: f["control"].__setitem__(0, 9), 201),
    ("eos-range", lambda f: f["control"].__setitem__(2, W.dims.vocab), 201),
    ("dup-block", lambda f: f["table"].__setitem__((1, 0), 1), 203),
    ("block-range", lambda f: f["table"].__setitem__((0, 1), 8), 203),
    ("active-2", lambda f: f["active"].__setitem__(0, 2), 201),
    ("token-range", lambda f: f["tokens"].__setitem__(0, W.dims.vocab), 201),
    ("len-mismatch", lambda f: f["lengths"].__setitem__(0, 3), 201),
    ("capacity", lambda f: (f["positions"].__setitem__(0, CAP - 1), f["lengths"].__setitem__(0, CAP)), 202),
    ("slot-mismatch", lambda f: f["slots"].__setitem__(0, 5), 204),
    ("gen-zero-active", lambda f: f["control"].__setitem__(3 + B, 0), 201),
    ("continuity", lambda f: (f["positions"].__setitem__(0, 1), f["lengths"].__setitem__(0, 2)), 212),
]


@pytest.mark.parametrize("name,mutate,expected", FALLBACK_CASES, ids=[c[0] for c in FALLBACK_CASES])
def test_fallback_codes_match_oracle(rt, weights, name, mutate, expected):
    dec, ctl = oracle_controller(W, weights)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    table = FROZEN_TABLE.copy()
    f = {
        "tokens": np.array([5, 6, 7, 8], dtype=np.int64),
        "positions": np.zeros(B, dtype=np.int64),
        "lengths": np.ones(B, dtype=np.int32),
        "active": np.ones(B, dtype=np.int32),
        "table": table,
        "control": np.zeros(control_input_elements(B), dtype=np.int32),
    }
    f["control"][0] = 2
    f["control"][1 : 1 + B] = W.eos
    f["control"][3 + B : 3 + 2 * B] = np.arange(1, B + 1)
    f["slots"] = np.array([slot_of(table, r, 0, BS) for r in range(B)], dtype=np.int32)
    mutate(f)
    if name in ("capacity", "continuity", "len-mismatch"):
        f["slots"][0] = slot_of(table, 0, int(f["positions"][0]), BS) if f["positions"][0] < CAP else -1
    feed = pack_feed(f["tokens"], f["positions"], f["lengths"], f["slots"], f["active"], f["table"], tiling_bytes(), f["control"])
    hist, control = rt.proc(feed)
    ref = ctl.proc(EpochFeed(f["tokens"], f["positions"], f["lengths"], f["slots"], f["active"], f["table"].reshape(-1), tiling_bytes(), f["control"]))
    assert control[3] == expected, (name, control[3])
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(control, ref.control)


def test_bridge_execute_matches_oracle_bridge(rt, weights):
    """resident_epoch_execute on four new generations (pos 0, len 1) with the
    bridge's identity table, K=4."""
    dec, ctl = oracle_controller(W, weights)
    rt.write_state("key_cache", torch.zeros(rt.cache_bytes // 4, dtype=torch.float32))
    rt.write_state("value_cache", torch.zeros(rt.cache_bytes // 4, dtype=torch.float32))
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    tokens = [11, 22, 33, 44]
    out = rt.execute(4, 4, tokens, [0] * B, [1] * B, [W.eos] * B, [1, 2, 3, 4])
    assert out.status == 0 and out.commit_state == 2 and out.feed_calls == 1 and out.fetch_calls == 1
    assert out.declared_input_bytes == 260 and out.declared_output_bytes == 368
    hist = np.full((8, B), -1, dtype=np.int64)
    for r in range(B):
        hist[: out.executed[r], r] = out.token_ids[r, : out.executed[r]]
    ctl.token_override = TeacherForcing(hist, rel_tol(W.dims))
    ref = obridge.execute(ctl, 4, 4, tokens, [0] * B, [1] * B, [W.eos] * B, [1, 2, 3, 4], tiling_bytes(), configured_eos=W.eos)
    assert not ctl.token_override.mismatches
    np.testing.assert_array_equal(out.token_ids.reshape(-1), ref.token_ids)
    np.testing.assert_array_equal(out.executed, ref.executed)
    np.testing.assert_array_equal(out.row_generations, ref.row_generations)
    assert out.model_calls == ref.model_calls and out.device_status == ref.device_status


def test_bridge_validation_codes(rt):
    assert rt.execute(0, 2, [0] * B, [0] * B, [1] * B, [1] * B, [1, 0, 0, 0]).status == 10
    assert rt.execute(1, 9, [0] * B, [0] * B, [1] * B, [1] * B, [1, 0, 0, 0]).status == 10
    bad_len = rt.execute(1, 2, [0] * B, [0] * B, [2] * B, [1] * B, [1, 0, 0, 0])
    assert bad_len.status == 11 and bad_len.commit_state == 0
    assert rt.execute(2, 2, [0] * B, [0] * B, [1] * B, [1] * B, [1, 0, 0, 0]).status == 12
