"""The epoch-controller oracle against known answers (CPU only).

Every expectation below is derived by hand from the closed forms of
controller/g4c_b4_resident_epoch.cpp ("CTRL") -- validation order 335-385,
generation continuity 448-471, the K-step loop 485-590, finish reasons
592-597, ``emit`` 296-324 -- using a stub decoder whose greedy token is a
known function of its input, so no expectation re-runs the oracle's own
formula.  The import checksum is checked against a restatement of the
reference's host-side ``kv_payload_checksum``
(src/vllm_ascend_resident_epoch/kv_transfer.py:159-174, zlib.adler32 over the
imported blocks), a different code path from CTRL's device checksum
(CTRL:149-163, 430-445) that must agree with it.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from oracle.controller import (
    FINISH_ALREADY,
    FINISH_EMPTY,
    FINISH_EOS,
    FINISH_FALLBACK,
    FINISH_MAX_STEPS,
    IMPORT_GRAPH_FLAG,
    STATUS_CAPACITY_EXCEEDED,
    STATUS_INVALID_BLOCK_TABLE,
    STATUS_INVALID_METADATA,
    STATUS_NON_FINITE_LOGITS,
    STATUS_OK,
    STATUS_POSITION_PROGRESS,
    STATUS_RESIDENT_CONTINUITY,
    STATUS_SLOT_MISMATCH,
    STATUS_UNSUPPORTED_GRAPH,
    STATUS_UNSUPPORTED_SAMPLING,
    ControllerGeometry,
    EpochController,
    EpochFeed,
    adler32_update,
    argmax_finite,
    compute_slot,
    control_input_elements,
    control_output_elements,
)

B, V, LAYERS, KVH, D = 4, 64, 2, 1, 2
GEO = ControllerGeometry(batch=B, capacity=8, physical_blocks=8, blocks_per_row=2, block_size=4, vocab=V, num_layers=LAYERS)
CACHE_SHAPE = (LAYERS, GEO.physical_blocks, GEO.block_size, KVH, D)
TILING = bytes(72)


def successor(token: int) -> int:
    """The stub decoder's greedy token."""
    return (7 * token + 3) % V


class StubDecoder:
    """Decoder-ABI stub: logits one-hot at ``successor(token)``; the KV slot of
    each active row receives ``token + 1`` in every layer; ``next_position`` as
    DEC:409-411.  ``nan_call``/``stall_call`` plant a non-finite logit or a
    stalled position at one call."""

    def __init__(self, nan_call: int | None = None, stall_call: int | None = None):
        self.calls = 0
        self.nan_call = nan_call
        self.stall_call = stall_call
        self.inputs: list[dict] = []

    def __call__(self, token, position, length, table, slot, key, value, tiling, active, *, inplace=False):
        if not inplace:
            key, value = key.clone(), value.clone()
        self.inputs.append({"token": token.clone(), "position": position.clone(), "length": length.clone(), "slot": slot.clone(), "active": active.clone()})
        logits = torch.zeros(B, 1, V)
        slots = GEO.physical_blocks * GEO.block_size
        for r in range(B):
            logits[r, 0, successor(int(token[r, 0]))] = 1.0
            s = int(slot[r])
            if int(active[r]) and 0 <= s < slots:
                key[:, s // GEO.block_size, s % GEO.block_size] = float(int(token[r, 0]) + 1)
                value[:, s // GEO.block_size, s % GEO.block_size] = -float(int(token[r, 0]) + 1)
        if self.calls == self.nan_call:
            logits[0, 0, 5] = float("nan")
        nxt = torch.where(active.to(torch.bool), position + 1, position)
        if self.calls == self.stall_call:
            nxt = position.clone()
        self.calls += 1
        return logits, key, value, nxt


def make_controller(model=None) -> EpochController:
    return EpochController(GEO, model or StubDecoder(), CACHE_SHAPE, torch.float32)


def control(K=8, eos=(V - 1,) * B, sampling=0, variant=0, gens=(1, 2, 0, 0)) -> np.ndarray:
    return np.array([K, *eos, sampling, variant, *gens], dtype=np.int32)


def identity_table() -> np.ndarray:
    return np.arange(B * GEO.blocks_per_row, dtype=np.int32)


def make_feed(
    tokens=(10, 20, 0, 30),
    positions=(0, 0, 0, 2),
    lengths=(1, 1, 0, 3),
    active=(1, 1, 0, 0),
    table=None,
    slots=None,
    ctl=None,
    payload=None,
) -> EpochFeed:
    table = identity_table() if table is None else np.asarray(table, dtype=np.int32)
    if slots is None:
        slots = [compute_slot(GEO, table, r, positions[r]) for r in range(B)]
    return EpochFeed(
        token=np.asarray(tokens, dtype=np.int64),
        position=np.asarray(positions, dtype=np.int64),
        sequence_length=np.asarray(lengths, dtype=np.int32),
        slot_mapping=np.asarray(slots, dtype=np.int32),
        active_mask=np.asarray(active, dtype=np.int32),
        block_table=table,
        tiling=TILING,
        control=control() if ctl is None else ctl,
        import_payload=payload,
    )


def offsets() -> dict[str, int]:
    """CTRL:28-38 at B=4, written out."""
    return {"eos": 6, "initial_active": 10, "executed": 14, "reason": 18, "initial_count": 22, "final_count": 23, "generation": 24}


def test_control_layout_matches_reference_constants():
    # CTRL:28-29: 1 + B + 2 + B inputs, 6 + 4B + 2 + B outputs (11 and 28 at B=4,
    # src/vllm_ascend_resident_epoch/abi.py:26,30).
    assert control_input_elements(4) == 11
    assert control_output_elements(4) == 28
    o = offsets()
    assert (GEO.eos_off, GEO.initial_active_off, GEO.executed_off, GEO.reason_off) == (o["eos"], o["initial_active"], o["executed"], o["reason"])
    assert (GEO.initial_count_off, GEO.final_count_off, GEO.generation_off) == (o["initial_count"], o["final_count"], o["generation"])


# --------------------------------------------------------------------------
# helpers of the oracle
# --------------------------------------------------------------------------
def test_compute_slot_closed_form():
    table = np.array([5, 2, 7, 0, 1, 6, 3, 4], dtype=np.int32)
    g = ControllerGeometry(batch=4, capacity=8, physical_blocks=8, blocks_per_row=2, block_size=4, vocab=V, num_layers=1)
    # row 1, position 6: logical block 1 -> table[1*2+1] = 0 -> slot 0*4 + 2
    assert compute_slot(g, table, 1, 6) == 2
    # row 2, position 3: logical block 0 -> table[4] = 1 -> slot 4 + 3
    assert compute_slot(g, table, 2, 3) == 7
    for bad in ((-1, 0), (4, 0), (0, -1), (0, 8)):
        assert compute_slot(g, table, *bad) == -1
    broken = table.copy()
    broken[0] = 8  # physical block out of range
    assert compute_slot(g, broken, 0, 0) == -1


def test_argmax_finite_first_max_and_non_finite():
    rng = np.random.default_rng(1)
    for _ in range(200):
        row = rng.integers(-3, 4, size=37).astype(np.float32)  # many ties
        brute = min(i for i in range(len(row)) if row[i] == row.max())
        assert argmax_finite(row) == brute
    row = np.zeros(9, dtype=np.float32)
    for bad in (np.nan, np.inf, -np.inf):
        row2 = row.copy()
        row2[4] = bad
        assert argmax_finite(row2) is None


@pytest.mark.parametrize("size", [0, 1, 5551, 5552, 5553, 3 * 5552 + 17, 100_000])
def test_adler32_update_matches_zlib(size):
    data = np.random.default_rng(size).integers(0, 256, size=size, dtype=np.uint8).tobytes()
    first, second = adler32_update(data, 1, 0)
    assert ((second << 16) | first) == zlib.adler32(data)
    # chained updates equal one pass over the concatenation
    cut = size // 3
    f1, s1 = adler32_update(data[:cut], 1, 0)
    f2, s2 = adler32_update(data[cut:], f1, s1)
    assert ((s2 << 16) | f2) == zlib.adler32(data)


# --------------------------------------------------------------------------
# validation (CTRL:335-385): first failing check wins, every row FALLBACK
# --------------------------------------------------------------------------
def _fallback_case(name):
    tok, pos, length, act = [10, 20, 0, 30], [0, 0, 0, 2], [1, 1, 0, 3], [1, 1, 0, 0]
    table = identity_table()
    ctl = control()
    slots = None
    if name == "k_zero":
        ctl = control(K=0)
        return make_feed(ctl=ctl), STATUS_INVALID_METADATA
    if name == "k_nine":
        return make_feed(ctl=control(K=9)), STATUS_INVALID_METADATA
    if name == "sampling":
        return make_feed(ctl=control(sampling=1, variant=16)), STATUS_UNSUPPORTED_SAMPLING
    if name == "variant":
        return make_feed(ctl=control(variant=16)), STATUS_UNSUPPORTED_GRAPH
    if name == "eos_range":
        return make_feed(ctl=control(eos=(0, V, 0, 0))), STATUS_INVALID_METADATA
    if name == "table_duplicate":
        table = table.copy()
        table[3] = table[0]
        return make_feed(table=table, slots=[0, 8, 0, 0]), STATUS_INVALID_BLOCK_TABLE
    if name == "table_range":
        table = table.copy()
        table[5] = 8
        return make_feed(table=table, slots=[0, 8, 0, 0]), STATUS_INVALID_BLOCK_TABLE
    if name == "active_not_binary":
        act = [1, 2, 0, 0]
    elif name == "token_range":
        tok = [10, V, 0, 30]
    elif name == "position_range":
        pos, length = [0, 8, 0, 2], [1, 9, 0, 3]
    elif name == "active_without_generation":
        ctl = control(gens=(1, 0, 0, 0))
    elif name == "active_length":
        length = [1, 2, 0, 3]
    elif name == "capacity":
        pos, length = [0, 1, 0, 2], [1, 2, 0, 3]  # 1 + 8 > 8
    elif name == "empty_with_generation":
        ctl = control(gens=(1, 2, 5, 0))
    elif name == "inactive_length":
        length = [1, 1, 0, 2]
    elif name == "slot":
        slots = [0, 9, 16, 18]
        slots[1] = 0  # row 1 must be at block 2 (slot 8)
    else:
        raise KeyError(name)
    feed = make_feed(tokens=tok, positions=pos, lengths=length, active=act, table=table, slots=slots, ctl=ctl)
    expected = {"capacity": STATUS_CAPACITY_EXCEEDED, "slot": STATUS_SLOT_MISMATCH}.get(name, STATUS_INVALID_METADATA)
    return feed, expected


FALLBACK_CASES = [
    "k_zero", "k_nine", "sampling", "variant", "eos_range", "table_duplicate", "table_range",
    "active_not_binary", "token_range", "position_range", "active_without_generation",
    "active_length", "capacity", "empty_with_generation", "inactive_length", "slot",
]


@pytest.mark.parametrize("case", FALLBACK_CASES)
def test_validation_fallbacks(case):
    feed, status = _fallback_case(case)
    ctl = make_controller()
    fetch = ctl.proc(feed)
    c = fetch.control
    assert c[3] == status
    assert c[4] == 0  # no model call
    assert c[5] == 1  # non-import: 1 on fallback (CTRL:301-303)
    assert (fetch.history == -1).all()
    assert list(c[18:22]) == [FINISH_FALLBACK] * B
    assert list(c[14:18]) == [0] * B
    assert c[0] == int(feed.control[0]) and c[1] == int(feed.control[1 + B])
    assert list(c[6:10]) == list(feed.control[1 : 1 + B])
    assert list(c[10:14]) == list(feed.active_mask)
    assert c[22] == int(np.count_nonzero(feed.active_mask)) and c[23] == c[22]


# --------------------------------------------------------------------------
# the K-step loop
# --------------------------------------------------------------------------
def chain(token: int, n: int) -> list[int]:
    out = []
    for _ in range(n):
        token = successor(token)
        out.append(token)
    return out


def test_epoch_eos_max_steps_empty_and_finished_rows():
    eos1 = chain(20, 2)[-1]  # row 1 stops at its second token
    ctl = make_controller()
    fetch = ctl.proc(make_feed(ctl=control(eos=(V - 1, eos1, 0, 0))))
    c, h = fetch.control, fetch.history
    assert c[3] == STATUS_OK and c[5] == 0 and c[4] == 8
    assert list(h[:, 0]) == chain(10, 8)
    assert list(h[:2, 1]) == chain(20, 2) and (h[2:, 1] == -1).all()
    assert (h[:, 2:] == -1).all()
    assert list(c[14:18]) == [8, 2, 0, 0]  # executed
    assert list(c[18:22]) == [FINISH_MAX_STEPS, FINISH_EOS, FINISH_EMPTY, FINISH_ALREADY]
    assert c[22] == 2 and c[23] == 1  # initial / final active counts
    assert list(c[24:28]) == [1, 2, 0, 0]  # generations echoed for active rows only
    # resident rows (CTRL:599-614): where each row stands after the epoch
    assert ctl.resident_generation[:2] == [1, 2]
    assert ctl.resident_token[:2] == [chain(10, 8)[-1], eos1]
    assert ctl.resident_position[:2] == [8, 2] and ctl.resident_length[:2] == [9, 3]


def test_epoch_model_inputs_follow_the_rows():
    model = StubDecoder()
    ctl = make_controller(model)
    ctl.proc(make_feed(ctl=control(K=3)))
    assert model.calls == 3
    second = model.inputs[1]
    # after one step row 0 feeds its first token at position 1, slot = block 0 offset 1
    assert int(second["token"][0, 0]) == successor(10)
    assert int(second["position"][0]) == 1 and int(second["length"][0, 0]) == 2
    assert int(second["slot"][0]) == 1 and int(second["slot"][1]) == 2 * GEO.block_size + 1
    assert list(second["active"]) == [1, 1, 0, 0]
    # inactive rows keep their feed values
    assert int(second["position"][3]) == 2 and int(second["slot"][3]) == compute_slot(GEO, identity_table(), 3, 2)


def test_epoch_stops_when_all_rows_finish():
    eos = (successor(10), successor(20), 0, 0)
    ctl = make_controller()
    fetch = ctl.proc(make_feed(ctl=control(eos=eos)))
    assert fetch.control[4] == 1  # one model call, then no active row
    assert list(fetch.control[18:20]) == [FINISH_EOS, FINISH_EOS]


def test_cache_adoption_and_row_clear_on_new_generation():
    ctl = make_controller()
    ctl.proc(make_feed(ctl=control(K=2)))
    k = ctl.resident_key
    # row 0 wrote token+1 at slots 0, 1 of block 0; row 1 at block 2
    assert float(k[0, 0, 0, 0, 0]) == 11 and float(k[0, 0, 1, 0, 0]) == successor(10) + 1
    assert float(k[1, 2, 0, 0, 0]) == 21
    # continue row 0 (same generation), restart row 1 with generation 3
    t0 = chain(10, 2)[-1]
    feed = make_feed(tokens=(t0, 40, 0, 30), positions=(2, 0, 0, 2), lengths=(3, 1, 0, 3), ctl=control(K=1, gens=(1, 3, 0, 0)))
    fetch = ctl.proc(feed)
    assert fetch.control[3] == STATUS_OK
    k = ctl.resident_key
    assert float(k[0, 0, 0, 0, 0]) == 11  # row 0 kept
    assert float(k[0, 0, 2, 0, 0]) == t0 + 1
    assert float(k[0, 2, 0, 0, 0]) == 41  # row 1 cleared, then written
    assert float(k[0, 2, 1, 0, 0]) == 0.0


@pytest.mark.parametrize(
    "tokens,positions,lengths,gens",
    [
        ((99 % V, 20, 0, 30), (2, 0, 0, 2), (3, 1, 0, 3), (1, 2, 0, 0)),  # same generation, wrong token
        (None, (3, 0, 0, 2), (4, 1, 0, 3), (1, 2, 0, 0)),  # same generation, wrong position
        ((5, 20, 0, 30), (2, 0, 0, 2), (3, 1, 0, 3), (7, 2, 0, 0)),  # new generation not at position 0
    ],
)
def test_resident_continuity_fallback(tokens, positions, lengths, gens):
    ctl = make_controller()
    ctl.proc(make_feed(ctl=control(K=2)))
    if tokens is None:
        tokens = (chain(10, 2)[-1], 20, 0, 30)
    key_before = ctl.resident_key.clone()
    rows_before = (list(ctl.resident_token), list(ctl.resident_position))
    fetch = ctl.proc(make_feed(tokens=tokens, positions=positions, lengths=lengths, ctl=control(K=1, gens=gens)))
    assert fetch.control[3] == STATUS_RESIDENT_CONTINUITY
    assert torch.equal(ctl.resident_key, key_before)
    assert (list(ctl.resident_token), list(ctl.resident_position)) == rows_before


def test_non_finite_logits_fallback_keeps_resident_state():
    ctl = make_controller(StubDecoder(nan_call=2))
    fetch = ctl.proc(make_feed())
    assert fetch.control[3] == STATUS_NON_FINITE_LOGITS
    assert fetch.control[4] == 3  # the failing call counts
    assert list(fetch.control[18:22]) == [FINISH_FALLBACK] * B
    # the epoch's cache writes are discarded (CTRL:583-584, 599-600)
    assert float(ctl.resident_key.abs().sum()) == 0.0
    assert ctl.resident_valid == [0] * B


def test_position_progress_fallback():
    ctl = make_controller(StubDecoder(stall_call=1))
    fetch = ctl.proc(make_feed())
    assert fetch.control[3] == STATUS_POSITION_PROGRESS
    assert fetch.control[4] == 2


# --------------------------------------------------------------------------
# KV import (CTRL:387-446)
# --------------------------------------------------------------------------
def payload_checksum(payload: bytes, mask: int) -> int:
    """src/vllm_ascend_resident_epoch/kv_transfer.py:159-174 restated:
    zlib.adler32 over [cache K, V][layer][row in mask] blocks of the payload."""
    block_bytes = GEO.block_size * KVH * D * 4
    cache_bytes = LAYERS * B * block_bytes
    checksum = 1
    for base in (0, cache_bytes):
        for layer in range(LAYERS):
            for row in range(B):
                if mask & (1 << row):
                    off = base + (layer * B + row) * block_bytes
                    checksum = zlib.adler32(payload[off : off + block_bytes], checksum)
    return checksum & 0xFFFFFFFF


def test_import_adopts_blocks_and_checksum_matches_host_payload_checksum():
    rng = np.random.default_rng(7)
    n = 2 * LAYERS * B * GEO.block_size * KVH * D
    payload = rng.standard_normal(n).astype(np.float32).tobytes()
    mask = 0b0010
    ctl = make_controller()
    # row 1 imports at position 3 (prefix of 3 tokens already in the payload)
    feed = make_feed(tokens=(10, 33, 0, 30), positions=(0, 3, 0, 2), lengths=(1, 4, 0, 3),
                     ctl=control(K=1, variant=IMPORT_GRAPH_FLAG | mask), payload=payload)
    fetch = ctl.proc(feed)
    c = fetch.control
    assert c[3] == STATUS_OK
    assert int(np.uint32(np.int32(c[5]))) == payload_checksum(payload, mask)
    assert c[2] == 0  # the graph variant without the import bits
    src = np.frombuffer(payload, dtype=np.float32).reshape(2, LAYERS, B, GEO.block_size, KVH, D)
    dest = int(identity_table()[1 * GEO.blocks_per_row])
    got = ctl.resident_key[:, dest].numpy()
    # positions 0..2 keep the imported prefix; position 3 was written by the step
    assert np.array_equal(got[:, :3], src[0, :, 1, :3])
    assert float(ctl.resident_key[0, dest, 3, 0, 0]) == 34


@pytest.mark.parametrize(
    "mask,status",
    [
        (0, STATUS_INVALID_METADATA),  # CTRL:388-389
        # bit 4 is outside the low nibble the variant decode strips
        # (CTRL:214-217), so it reads as graph variant 16: 206 comes first
        (1 << B, STATUS_UNSUPPORTED_GRAPH),
    ],
)
def test_import_mask_out_of_range(mask, status):
    n = 2 * LAYERS * B * GEO.block_size * KVH * D
    feed = make_feed(ctl=control(variant=IMPORT_GRAPH_FLAG | mask), payload=bytes(4 * n))
    assert make_controller().proc(feed).control[3] == status


def test_import_requires_active_row_with_generation():
    n = 2 * LAYERS * B * GEO.block_size * KVH * D
    feed = make_feed(ctl=control(variant=IMPORT_GRAPH_FLAG | 0b0100), payload=bytes(4 * n))  # row 2 is empty
    assert make_controller().proc(feed).control[3] == STATUS_INVALID_METADATA
