"""GPU parity at the reference's own geometry and window: the full
Qwen2.5-7B shape, B=4, 8 blocks of 128 slots, 2 blocks per row and the
reference's logical capacity of 8 (batched_decoder_step.py:33,
controller/g4c_b4_resident_epoch.cpp:18), created from a graph
configuration in the reference's own format (config/graph_config.json: the
decoder's nine input descriptors) plus a synthetic-weights source.

Checked against the oracle at capacity 8: an epoch that ends exactly at the
window (pos + K == 8), status 202 when pos + K > 8 (CTRL:368-369) through
the 8-input ABI and status 11 through the bridge call
(resident_epoch_bridge.cpp:539-546), and every validation fallback code of
CTRL:335-385.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from cruise_amd.runtime import ResidentEpochRuntime, pack_feed, tiling_bytes
from oracle.controller import EpochFeed, control_input_elements
from oracle.decoder import PagedGeometry, inv_freq, weight_shapes
from oracle.workloads import C3, Workload, identity_table, slot_of
from parity import TeacherForcing, assert_close_rel, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = Workload("qwen7b-window8", C3.dims, PagedGeometry(batch=4, physical_blocks=8, block_size=128, blocks_per_row=2,
                                                       window=8), eos=151645, seed=C3.seed + 8)
B = W.geometry.batch
BS = W.geometry.block_size
CAP = 8

REFERENCE_GRAPH_CONFIG = {
    "build_options": {"ge.externalWeight": "1", "ge.modelFileNamePrefix": "attempt71_b4_decoder"},
    "inputs_tensor_desc": [
        {"data_type": "DT_INT64", "shape": [4, 1]},
        {"data_type": "DT_INT64", "shape": [4]},
        {"data_type": "DT_INT32", "shape": [4, 1]},
        {"data_type": "DT_BFLOAT16", "shape": [28, 8, 128, 4, 128]},
        {"data_type": "DT_INT32", "shape": [4]},
        {"data_type": "DT_INT32", "shape": [4]},
        {"data_type": "DT_INT32", "shape": [4, 2]},
        {"data_type": "DT_BFLOAT16", "shape": [28, 8, 128, 4, 128]},
        {"data_type": "DT_UINT8", "shape": [72]},
    ],
}


@pytest.fixture(scope="module")
def rt_weights(tmp_path_factory):
    cfg = dict(REFERENCE_GRAPH_CONFIG)
    cfg["weights"] = {"source": "synthetic", "seed": W.seed, "std": 0.02}
    cfg["engine"] = {"require_dev_shm": False}
    path = tmp_path_factory.mktemp("compat8") / "graph_config.json"
    path.write_text(json.dumps(cfg))
    rt = ResidentEpochRuntime(None, graph_config=str(path))
    assert rt.info("capacity") == CAP and rt.info("physical_blocks") == 8 and rt.info("layers") == 28
    rt.write_state("inv_freq", inv_freq(W.dims).contiguous())
    cpu = {}
    for name, shape in weight_shapes(W.dims).items():
        t = torch.empty(shape, dtype=torch.bfloat16)
        rt.read_state(name, t)
        cpu[name] = t
    yield rt, cpu
    rt.close()


def reset(rt):
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))


def test_epoch_to_the_end_of_the_window(rt_weights):
    """Prompts of 2-5 tokens, then the largest K with pos + K <= 8 for every
    row: the last step writes slot 7 and the row's next slot is -1."""
    rt, cpu = rt_weights
    reset(rt)
    rng = np.random.default_rng(W.seed)
    table = identity_table(B, W.geometry.blocks_per_row)
    ps = [list(map(int, rng.integers(0, W.dims.vocab, size=n))) for n in (4, 3, 2, 4)]
    _, ctl = oracle_controller(W, cpu)
    gens = np.arange(1, B + 1, dtype=np.int32)
    for r in range(B):
        rt.prefill(r, int(gens[r]), ps[r], table[r])
        ctl.prefill_row(r, int(gens[r]), ps[r], table[r])
    tokens = np.array([p[-1] for p in ps], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
    K = 4  # max position 3 + 4 == 8
    lengths = (positions + 1).astype(np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[3 + B :] = gens
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    act = np.ones(B, dtype=np.int32)
    hist, ctrl = rt.proc(pack_feed(tokens, positions, lengths, slots, act, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, act, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches, tf.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    assert ctrl[3] == 0 and ctrl[4] == K
    rows = rt.resident_rows()
    assert rows[2][0] == 7 and rows[3][0] == 8  # row 0 ends on the window's last slot
    for name, r in (("key_cache", ctl.resident_key), ("value_cache", ctl.resident_value)):
        got = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
        rt.read_state(name, got)
        assert_close_rel(got.view_as(r), r, rel_tol(W.dims), f"resident {name}")
    # two steps more do not fit rows at position 7: 202 on the device, 11 at
    # the bridge
    control[0] = 2
    positions2 = rows[2].astype(np.int64)
    lengths2 = (positions2 + 1).astype(np.int32)
    slots2 = np.array([slot_of(table, r, int(positions2[r]), BS) for r in range(B)], dtype=np.int32)
    tokens2 = rows[1].astype(np.int64)
    hist, ctrl = rt.proc(pack_feed(tokens2, positions2, lengths2, slots2, act, table, tiling_bytes(), control))
    ref = ctl.proc(EpochFeed(tokens2, positions2, lengths2, slots2, act, table.reshape(-1), tiling_bytes(), control))
    assert ctrl[3] == 202
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    out = rt.execute(4, 2, tokens2, positions2, lengths2, [W.eos] * B, gens)
    assert out.status == 11 and out.commit_state == 0


def base_feed():
    table = identity_table(B, W.geometry.blocks_per_row)
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
    return f


def pos_len(f, row, pos):
    f["positions"][row] = pos
    f["lengths"][row] = pos + 1


FALLBACKS = [
    ("sampling", lambda f: f["control"].__setitem__(1 + B, 1), 205),
    ("variant", lambda f: f["control"].__setitem__(2 + B, 7), 206),
    ("k-zero", lambda f: f["control"].__setitem__(0, 0), 201),
    ("k-nine", lambda f: f["control"].__setitem__(0, 9), 201),
    ("eos-range", lambda f: f["control"].__setitem__(3, W.dims.vocab), 201),
    ("dup-block", lambda f: f["table"].__setitem__((2, 1), 0), 203),
    ("block-range", lambda f: f["table"].__setitem__((3, 1), 8), 203),
    ("active-2", lambda f: f["active"].__setitem__(1, 2), 201),
    ("token-range", lambda f: f["tokens"].__setitem__(2, W.dims.vocab), 201),
    ("position-8", lambda f: pos_len(f, 0, 8), 201),
    ("len-mismatch", lambda f: f["lengths"].__setitem__(0, 3), 201),
    ("capacity-7+2", lambda f: pos_len(f, 3, 7), 202),
    ("capacity-6+4", lambda f: (pos_len(f, 1, 6), f["control"].__setitem__(0, 4)), 202),
    ("slot-mismatch", lambda f: f["slots"].__setitem__(2, 5), 204),
    ("empty-with-generation", lambda f: (f["active"].__setitem__(3, 0), f["lengths"].__setitem__(3, 0)), 201),
    ("gen-zero-active", lambda f: f["control"].__setitem__(3 + B, 0), 201),
    ("continuity", lambda f: pos_len(f, 0, 1), 212),
]


@pytest.mark.parametrize("name,mutate,expected", FALLBACKS, ids=[c[0] for c in FALLBACKS])
def test_fallback_codes_at_window_8(rt_weights, name, mutate, expected):
    rt, cpu = rt_weights
    _, ctl = oracle_controller(W, cpu)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    f = base_feed()
    f["slots"] = np.zeros(B, dtype=np.int32)
    mutate(f)
    table = f["table"]
    for r in range(B):
        if name != "slot-mismatch" or r != 2:
            p = int(f["positions"][r])
            f["slots"][r] = slot_of(table, r, p, BS) if 0 <= p < CAP and 0 <= table[r, p // BS] < 8 else -1
    feed = pack_feed(f["tokens"], f["positions"], f["lengths"], f["slots"], f["active"], table, tiling_bytes(),
                     f["control"])
    hist, control = rt.proc(feed)
    ref = ctl.proc(EpochFeed(f["tokens"], f["positions"], f["lengths"], f["slots"], f["active"], table.reshape(-1),
                             tiling_bytes(), f["control"]))
    assert control[3] == expected, (name, control[3])
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(control, ref.control)
