"""GPU parity of the batched prefill (resident_epoch_prefill_batch).

The batched prefill must leave the state the oracle's teacher-forced
prefill leaves (oracle/controller.py ``prefill_row``: clear the row's blocks,
decoder steps at positions 0..L-2, resident record token prompt[L-1],
position L-1, length L): written K/V at the model's tolerance, every other
slot untouched, the resident rows exact, and the epoch that follows equal to
the oracle's (teacher forced where the top-2 margin is not decisive).

* tiny fp32 model (FMA GEMM, per-token attention), prompts of 1-29 tokens;
* one Qwen2.5-7B layer in bf16 (MFMA GEMMs and MFMA attention), prompts of
  1-70 tokens against the oracle, and prompts of up to 250 tokens (four
  64-query tiles) against the engine's own single-row prefill, which the
  oracle pins above.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from cruise_amd.runtime import pack_feed, tiling_bytes
from oracle.controller import EpochFeed, control_input_elements
from oracle.weights import generate_weights
from oracle.decoder import PagedGeometry
from oracle.workloads import C1, C2, random_tables, slot_of
from parity import TeacherForcing, assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu


def reset(rt, dtype, B):
    elems = rt.cache_bytes // (2 if dtype == torch.bfloat16 else 4)
    zeros = torch.zeros(elems, dtype=dtype, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))


def read_caches(rt, dtype):
    elems = rt.cache_bytes // (2 if dtype == torch.bfloat16 else 4)
    k = torch.zeros(elems, dtype=dtype)
    v = torch.zeros(elems, dtype=dtype)
    rt.read_state("key_cache", k)
    rt.read_state("value_cache", v)
    return k, v


def written_slots(table, prompts, bs):
    out = []
    for r, p in enumerate(prompts):
        out += [slot_of(table, r, q, bs) for q in range(len(p) - 1)]
    return out


def check_caches(W, got, ref, slots, what):
    d = W.dims
    flat = lambda t: t.reshape(d.num_layers, -1, d.num_kv_heads, d.head_dim)
    mask = torch.ones(flat(got).shape[1], dtype=torch.bool)
    mask[slots] = False
    assert torch.equal(flat(got)[:, mask], flat(ref)[:, mask]), f"{what}: slots outside the prompts changed"
    assert_close_rel(flat(got)[:, slots], flat(ref)[:, slots], rel_tol(d), f"prefilled {what}")


def epoch_after_prefill(W, rt, ctl, table, prompts, gens, K):
    B = W.geometry.batch
    tokens = np.array([p[-1] for p in prompts], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in prompts], dtype=np.int64)
    lengths = (positions + 1).astype(np.int32)
    active = np.ones(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[3 + B : 3 + 2 * B] = gens
    slots = np.array([slot_of(table, r, int(positions[r]), W.geometry.block_size) for r in range(B)], dtype=np.int32)
    hist, ctrl = rt.proc(pack_feed(tokens, positions, lengths, slots, active, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches, tf.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    assert ctrl[3] == 0


def run_against_oracle(W, weights_dev, weights_cpu, lengths, seed, K, tuning=None):
    B = W.geometry.batch
    dtype = W.dims.torch_dtype
    rng = np.random.default_rng(seed)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    prompts = [list(map(int, rng.integers(0, W.dims.vocab, size=n))) for n in lengths]
    gens = np.arange(1, B + 1, dtype=np.int32) + seed % 1000
    rt = make_runtime(W, weights_dev, tuning=tuning)
    try:
        _, ctl = oracle_controller(W, weights_cpu)
        reset(rt, dtype, B)
        print(f"prefill_batch {W.name}: prompt lengths {lengths}", flush=True)
        rt.prefill_batch(list(range(B)), gens, prompts, table)
        torch.cuda.synchronize()
        for r in range(B):
            ctl.prefill_row(r, int(gens[r]), prompts[r], table[r])
        k, v = read_caches(rt, dtype)
        slots = written_slots(table, prompts, W.geometry.block_size)
        check_caches(W, k.view_as(ctl.resident_key), ctl.resident_key, slots, "keys")
        check_caches(W, v.view_as(ctl.resident_value), ctl.resident_value, slots, "values")
        rows = rt.resident_rows()
        assert list(rows[0]) == list(gens)
        assert list(rows[1]) == [p[-1] for p in prompts]
        assert list(rows[2]) == [len(p) - 1 for p in prompts] and list(rows[3]) == [len(p) for p in prompts]
        assert list(rows[4]) == [1] * B
        epoch_after_prefill(W, rt, ctl, table, prompts, gens, K)
    finally:
        rt.close()


def test_tiny_fp32_prefill_matches_oracle():
    w = generate_weights(C1.dims, C1.seed)
    run_against_oracle(C1, w, w, [1, 7, 20, 29], seed=5101, K=2)


@pytest.fixture(scope="module")
def c2_weights():
    dev = generate_weights(C2.dims, C2.seed, device="cuda")
    return dev, {k: v.cpu() for k, v in dev.items()}


def test_bf16_layer_prefill_matches_oracle(c2_weights):
    dev, cpu = c2_weights
    run_against_oracle(C2, dev, cpu, [41, 5, 70, 1], seed=5102, K=4)


def test_bf16_layer_prefill_other_prompts_matches_oracle(c2_weights):
    """The same check on another seed (other prompts and block tables)."""
    dev, cpu = c2_weights
    run_against_oracle(C2, dev, cpu, [41, 5, 70, 1], seed=5104, K=4)


def test_bf16_two_layer_long_prompt_prefill_matches_oracle():
    """A 250-token prompt (four query tiles, the last one partial) beside
    130-, 3- and 1-token prompts on two Qwen2.5-7B layers: layer 1's keys and
    values depend on layer 0's prefill attention over the whole prompt, so
    the oracle's teacher-forced prefill pins the causal attention, not only
    the projections."""
    from oracle.decoder import ModelDims
    from oracle.workloads import C2_DIMS

    dims = replace(C2_DIMS, num_layers=2)
    W = replace(C2, name="qwen7b-2layer", dims=dims, seed=C2.seed + 2)
    dev = generate_weights(W.dims, W.seed, device="cuda")
    cpu = {k: v.cpu() for k, v in dev.items()}
    assert isinstance(W.dims, ModelDims)
    run_against_oracle(W, dev, cpu, [250, 130, 3, 1], seed=5106, K=4)


def test_bf16_layer_prefill_matches_single_row_prefill(c2_weights):
    """Prompts up to 250 tokens (four query tiles, partial last tile): the
    batched pass against the engine's own per-row decoder steps."""
    dev, _ = c2_weights
    W = C2
    B = W.geometry.batch
    rng = np.random.default_rng(5103)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    lengths = [250, 129, 64, 2]
    prompts = [list(map(int, rng.integers(0, W.dims.vocab, size=n))) for n in lengths]
    rt = make_runtime(W, dev)
    try:
        reset(rt, torch.bfloat16, B)
        print("single-row prefill, prompt lengths", lengths, flush=True)
        for r in range(B):
            rt.prefill(r, 20 + r, prompts[r], table[r])
        k_ref, v_ref = read_caches(rt, torch.bfloat16)
        rows_ref = rt.resident_rows().copy()
        reset(rt, torch.bfloat16, B)
        print("batched prefill, prompt lengths", lengths, flush=True)
        rt.prefill_batch(list(range(B)), [20 + r for r in range(B)], prompts, table)
        k, v = read_caches(rt, torch.bfloat16)
        slots = written_slots(table, prompts, W.geometry.block_size)
        check_caches(W, k, k_ref, slots, "keys")
        check_caches(W, v, v_ref, slots, "values")
        np.testing.assert_array_equal(rt.resident_rows(), rows_ref)
    finally:
        rt.close()


def test_bf16_layer_long_prompts_match_single_row_prefill(c2_weights):
    """1,500- and 700-token prompts (window 1,536: up to 24 key tiles per
    query tile, partial last tiles): the batched pass against the engine's
    own per-row decoder steps."""
    dev, _ = c2_weights
    W = replace(C2, name="qwen7b-1layer-long",
                geometry=PagedGeometry(batch=2, physical_blocks=32, block_size=128, blocks_per_row=12, window=1536))
    B = W.geometry.batch
    rng = np.random.default_rng(5105)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    prompts = [list(map(int, rng.integers(0, W.dims.vocab, size=n))) for n in (1500, 700)]
    rt = make_runtime(W, dev)
    try:
        reset(rt, torch.bfloat16, B)
        print("single-row prefill, prompt lengths", [len(p) for p in prompts], flush=True)
        for r in range(B):
            rt.prefill(r, 40 + r, prompts[r], table[r])
        k_ref, v_ref = read_caches(rt, torch.bfloat16)
        rows_ref = rt.resident_rows().copy()
        reset(rt, torch.bfloat16, B)
        print("batched prefill", flush=True)
        rt.prefill_batch(list(range(B)), [40 + r for r in range(B)], prompts, table)
        k, v = read_caches(rt, torch.bfloat16)
        slots = written_slots(table, prompts, W.geometry.block_size)
        check_caches(W, k, k_ref, slots, "keys")
        check_caches(W, v, v_ref, slots, "values")
        np.testing.assert_array_equal(rt.resident_rows(), rows_ref)
    finally:
        rt.close()


def test_prefill_batch_argument_checks():
    w = generate_weights(C1.dims, C1.seed)
    rt = make_runtime(C1, w)
    try:
        table = np.zeros((1, C1.geometry.blocks_per_row), dtype=np.int32)
        for rows, gens, prompts, tab in (
            ([4], [1], [[1, 2]], table),                      # row outside the batch
            ([0], [0], [[1, 2]], table),                      # generation not positive
            ([0], [1], [[C1.dims.vocab]], table),             # token outside the vocabulary
            ([0], [1], [list(range(33))], table),             # longer than the window
            ([0], [1], [[1, 2]], np.full((1, 2), 8, np.int32)),  # block outside the pool
        ):
            with pytest.raises(RuntimeError, match="-1"):
                rt.prefill_batch(rows, gens, prompts, tab)
        with pytest.raises(RuntimeError, match="-1"):
            rt.prefill_batch([1, 1], [1, 2], [[1], [2]], np.zeros((2, 2), np.int32))  # repeated row
        # one-token prompts: nothing to compute, the rows are adopted
        rt.prefill_batch([2], [9], [[17]], table)
        rows = rt.resident_rows()
        assert [rows[i][2] for i in range(5)] == [9, 17, 0, 1, 1]
    finally:
        rt.close()
