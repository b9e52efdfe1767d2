"""The oracle's prefill stand-in ``EpochController.prefill_row`` (CPU only).

The reference brings a prompt onto the device through stock-vLLM prefill and
a KV import: controller/g4c_b4_resident_epoch.cpp:387-429 ("CTRL") clears the
row's blocks, copies the prompt's KV in, and records the row's generation,
token, position and length from the feed; the epoch then continues from
token = prompt[L-1], position L-1, length L (CTRL:448-463).  ``prefill_row``
restates that with teacher-forced decoder steps over positions 0..L-2.

What pins it here, independently of the oracle's own decoder:

* the K (after RoPE) and V it leaves at the row's slots for positions
  0..L-2, in every layer, against HF ``Qwen2ForCausalLM`` eager's
  DynamicCache after the same L-1 tokens -- what the reference's acceptance
  gate compares (history/attempts/g4c-attempt69b-b4-eager/
  batched_decoder_step.py:477-518) -- at the gate tolerance, and bf16 bit
  for bit;
* exactly: the row's slots from position L-1 on are zero (the clear), every
  block the row does not own is untouched, the resident record is
  (generation, prompt[L-1], L-1, L, valid), and other rows' records are
  unchanged;
* the epoch that follows: a K=2 continuation on the prefilled row passes the
  continuity check and its two steps' logits equal HF's next two steps;
* planted mistakes -- one position too many or too few, a skipped block
  clear, a record one position off -- each fail.

The prompt crosses a block boundary under a random block table.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.controller import (
    STATUS_OK,
    ControllerGeometry,
    EpochController,
    EpochFeed,
    compute_slot,
)
from oracle.decoder import ModelDims, OracleDecoder, PagedGeometry
from oracle.hf_reference import build_hf_model, hf_incremental
from oracle.weights import seeded_cache
from oracle.workloads import random_tables

from test_oracle_decoder import GATE_BF16, GATE_FP32, TINY, sharp_weights

B, BS, BPR, POOL = 4, 16, 2, 12
GEO = PagedGeometry(batch=B, physical_blocks=POOL, block_size=BS, blocks_per_row=BPR, window=BS * BPR)
ROW, GEN = 2, 7
TABLE = random_tables(np.random.default_rng(20263), B, BPR, POOL)  # [B, BPR], distinct blocks
PROMPT = [int(t) for t in np.random.default_rng(5).integers(0, TINY["vocab"], size=21)]  # 20 positions: crosses 16
GATES = {"bf16": GATE_BF16, "fp32": GATE_FP32}


def dims(dtype: str) -> ModelDims:
    return ModelDims(dtype=dtype, **TINY)


def make_controller(dtype: str, weights: dict) -> EpochController:
    d = dims(dtype)
    dec = OracleDecoder(d, GEO, weights)
    cg = ControllerGeometry(
        batch=B, capacity=GEO.window, physical_blocks=POOL, blocks_per_row=BPR, block_size=BS, vocab=d.vocab, num_layers=d.num_layers
    )
    ctrl = EpochController(cg, dec.forward, dec.cache_shape(), d.torch_dtype)
    # Start from nonzero caches so a missed clear or a stray write shows.
    ctrl.resident_key, ctrl.resident_value = seeded_cache(dec.cache_shape(), 530041, d.torch_dtype)
    for r in range(B):
        if r != ROW:
            ctrl.resident_generation[r] = 10 + r
            ctrl.resident_token[r] = 100 + r
            ctrl.resident_position[r] = r
            ctrl.resident_length[r] = r + 1
            ctrl.resident_valid[r] = 1
    return ctrl


@pytest.fixture(scope="module")
def weights():
    return {dt: sharp_weights(dims(dt), 11) for dt in ("bf16", "fp32")}


@pytest.fixture(scope="module")
def hf(weights):
    """HF eager over the whole prompt plus two greedy steps: logits and the
    K/V written per step."""
    out = {}
    for dt in ("bf16", "fp32"):
        model = build_hf_model(dims(dt), weights[dt])
        tokens = list(PROMPT)
        logits, keys, values = hf_incremental(model, tokens)
        tokens.append(int(torch.argmax(logits[-1])))
        out[dt] = (hf_incremental(model, tokens), tokens)
    return out


def slot_of(position: int) -> tuple[int, int]:
    return int(TABLE[ROW, position // BS]), position % BS


def prefill_problems(ctrl: EpochController, before: tuple, hf_kv: tuple, gate: float, exact: bool) -> list[str]:
    """Every way the prefilled state differs from what stock prefill plus an
    import leaves (an empty list when it is right)."""
    key0, value0, records0 = before
    _, ref_keys, ref_values = hf_kv
    L = len(PROMPT)
    problems = []
    for p in range(L - 1):
        blk, off = slot_of(p)
        for name, cache, ref in (("key", ctrl.resident_key, ref_keys), ("value", ctrl.resident_value, ref_values)):
            ours, want = cache[:, blk, off], ref[p]
            scale = float(want.float().abs().max())
            err = float((ours.float() - want.float()).abs().max()) / scale
            if err > gate or (exact and not torch.equal(ours, want)):
                problems.append(f"{name} at position {p}: rel err {err:.2e}")
    for p in range(L - 1, BS * BPR):
        blk, off = slot_of(p)
        if ctrl.resident_key[:, blk, off].any() or ctrl.resident_value[:, blk, off].any():
            problems.append(f"position {p} not zero")
    others = [b for b in range(POOL) if b not in set(TABLE[ROW].tolist())]
    if not (torch.equal(ctrl.resident_key[:, others], key0[:, others]) and torch.equal(ctrl.resident_value[:, others], value0[:, others])):
        problems.append("a block the row does not own changed")
    records = records_of(ctrl)
    want = {r: records0[r] for r in range(B)}
    want[ROW] = (GEN, PROMPT[-1], L - 1, L, 1)
    for r in range(B):
        if records[r] != want[r]:
            problems.append(f"row {r} record {records[r]} != {want[r]}")
    return problems


def records_of(ctrl: EpochController) -> list[tuple]:
    return [
        (ctrl.resident_generation[r], ctrl.resident_token[r], ctrl.resident_position[r], ctrl.resident_length[r], ctrl.resident_valid[r])
        for r in range(B)
    ]


def run_prefill(dtype: str, weights: dict) -> tuple[EpochController, tuple]:
    ctrl = make_controller(dtype, weights[dtype])
    before = (ctrl.resident_key.clone(), ctrl.resident_value.clone(), records_of(ctrl))
    ctrl.prefill_row(ROW, GEN, PROMPT, TABLE[ROW])
    return ctrl, before


def test_prompt_crosses_a_block_boundary_under_a_random_table():
    assert len(PROMPT) - 1 > BS
    assert sorted(TABLE.ravel().tolist()) != list(range(B * BPR))  # not the identity table
    assert len(set(TABLE.ravel().tolist())) == B * BPR


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_prefill_row_leaves_hf_cache_and_the_import_record(weights, hf, dtype):
    ctrl, before = run_prefill(dtype, weights)
    (_, keys, values), _ = hf[dtype]
    problems = prefill_problems(ctrl, before, (None, keys, values), GATES[dtype], exact=dtype == "bf16")
    assert not problems, problems


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_epoch_after_prefill_continues_like_hf(weights, hf, dtype):
    ctrl, _ = run_prefill(dtype, weights)
    (ref_logits, _, _), tokens = hf[dtype]
    L = len(PROMPT)
    token = np.zeros(B, dtype=np.int64)
    position = np.zeros(B, dtype=np.int64)
    length = np.zeros(B, dtype=np.int32)
    active = np.zeros(B, dtype=np.int32)
    token[ROW], position[ROW], length[ROW], active[ROW] = PROMPT[-1], L - 1, L, 1
    table = TABLE.reshape(-1).astype(np.int32)
    cg = ctrl.geometry
    slot = np.array([compute_slot(cg, table, r, int(position[r])) for r in range(B)], dtype=np.int32)
    gens = [0] * B
    gens[ROW] = GEN
    feed = EpochFeed(
        token=token, position=position, sequence_length=length, slot_mapping=slot, active_mask=active,
        block_table=table, tiling=bytes(72),
        control=np.array([2, *([dims(dtype).vocab - 1] * B), 0, 0, *gens], dtype=np.int32),
    )
    fetch = ctrl.proc(feed)
    assert int(fetch.control[3]) == STATUS_OK
    assert fetch.history[0, ROW] == tokens[L] and fetch.history[1, ROW] == int(torch.argmax(ref_logits[L]))
    for step in range(2):
        ours = torch.from_numpy(ctrl.logits_trace[step][ROW])
        want = ref_logits[L - 1 + step]
        err = float((ours - want).abs().max()) / float(want.abs().max())
        assert err <= GATES[dtype], f"step {step}: rel err {err:.2e}"
        if dtype == "bf16":
            assert torch.equal(ours, want), f"step {step} not bit-identical to HF eager"


def _one_too_many(mp):
    mp.setattr(EpochController, "_prefill_positions", staticmethod(lambda prompt: range(len(prompt))))


def _one_too_few(mp):
    mp.setattr(EpochController, "_prefill_positions", staticmethod(lambda prompt: range(len(prompt) - 2)))


def _no_clear(mp):
    mp.setattr(EpochController, "_clear_row_blocks", lambda self, table_row: None)


def _record_off_by_one(mp):
    real = EpochController.prefill_row

    def wrong(self, row, generation, prompt, table_row):
        real(self, row, generation, prompt, table_row)
        self.resident_position[row] += 1

    mp.setattr(EpochController, "prefill_row", wrong)


PLANTS = {"one_position_too_many": _one_too_many, "one_position_too_few": _one_too_few, "block_clear_skipped": _no_clear, "record_position_off_by_one": _record_off_by_one}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_planted_prefill_mistake_is_caught(weights, hf, monkeypatch, plant):
    PLANTS[plant](monkeypatch)
    ctrl, before = run_prefill("bf16", weights)
    (_, keys, values), _ = hf["bf16"]
    assert prefill_problems(ctrl, before, (None, keys, values), GATE_BF16, exact=True), f"planted {plant} not detected"
