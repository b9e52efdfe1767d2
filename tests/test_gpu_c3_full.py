"""GPU parity at the full Qwen2.5-7B shape (28 layers, hidden 3584, 28/4
heads, head_dim 128, intermediate 18944, vocab 152064, bf16), B=4, block 128
x 2 blocks per row, capacity 256: the bench workload.

The engine generates its synthetic weights on the device; the oracle reads
the same bytes back.  Checked: one decoder step over a permuted block table
with seeded KV (logits, written KV, untouched KV, next positions), and two
consecutive K=8 epochs after prefilling 2-5 token prompts (history and control
record bit-exact with the teacher-forced oracle, resident caches at
tolerance), which exercises resident continuity across epochs at full size.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cruise_amd.runtime import ResidentEpochRuntime, WeightSpec, pack_feed, tiling_bytes
from oracle.controller import EpochFeed, control_input_elements
from oracle.decoder import inv_freq, weight_shapes
from oracle.weights import seeded_cache
from oracle.workloads import C3, slot_of
from parity import TeacherForcing, assert_close_rel, engine_config, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C3
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row


@pytest.fixture(scope="module")
def rt_weights():
    rt = ResidentEpochRuntime(engine_config(W, weights=WeightSpec("synthetic", W.seed, 0.02)))
    rt.write_state("inv_freq", inv_freq(W.dims).contiguous())
    cpu = {}
    for name, shape in weight_shapes(W.dims).items():
        t = torch.empty(shape, dtype=torch.bfloat16)
        rt.read_state(name, t)
        cpu[name] = t
    yield rt, cpu
    rt.close()


def test_full_model_decoder_step(rt_weights):
    rt, cpu = rt_weights
    rng = np.random.default_rng(303)
    table = rng.permutation(B * BPR).astype(np.int32).reshape(B, BPR)
    ctx = np.array([2, 130, 57, 5], dtype=np.int64)  # row 1 crosses into its second block
    pos = ctx.copy()
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = np.array([1, 1, 1, 1], dtype=np.int32)
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 530041, torch.bfloat16)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    gk, gv = key.clone().cuda(), value.clone().cuda()
    logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32, device="cuda")
    nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
    rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
    torch.cuda.synchronize()
    assert torch.equal(nxt.cpu(), ref_next)
    assert_close_rel(logits.cpu(), ref_logits.reshape(B, -1), rel_tol(W.dims), "logits")
    flat = lambda t: t.reshape(W.dims.num_layers, -1, W.dims.num_kv_heads, W.dims.head_dim)
    written = [int(s) for s in slot]
    mask = torch.ones(flat(key).shape[1], dtype=torch.bool)
    mask[written] = False
    for got, ref, inp, what in ((gk.cpu(), ref_k, key, "key"), (gv.cpu(), ref_v, value, "value")):
        assert torch.equal(flat(got)[:, mask], flat(inp)[:, mask]), f"unaddressed {what} slots changed"
        assert_close_rel(flat(got)[:, written], flat(ref)[:, written], rel_tol(W.dims), f"written {what}")
    for r in range(B):
        row = ref_logits[r, 0].numpy()
        top2 = np.sort(row)[-2:]
        if top2[1] - top2[0] > rel_tol(W.dims) * np.abs(row).max():
            assert int(logits[r].argmax()) == int(row.argmax())


def run_epoch(rt, ctl, tokens, positions, gens, table, K=8):
    lengths = (positions + 1).astype(np.int32)
    active = np.ones(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[3 + B :] = gens
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    hist, ctrl = rt.proc(pack_feed(tokens, positions, lengths, slots, active, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches, tf.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    return hist, ctrl


def test_full_model_two_epochs_after_prefill(rt_weights):
    rt, cpu = rt_weights
    rng = np.random.default_rng(W.seed)
    table = np.arange(B * BPR, dtype=np.int32).reshape(B, BPR)
    ps = [list(map(int, rng.integers(0, W.dims.vocab, size=int(rng.integers(2, 6))))) for _ in range(B)]
    _, ctl = oracle_controller(W, cpu)
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    gens = np.arange(1, B + 1, dtype=np.int32)
    for r in range(B):
        rt.prefill(r, int(gens[r]), ps[r], table[r])
        ctl.prefill_row(r, int(gens[r]), ps[r], table[r])
    tokens = np.array([p[-1] for p in ps], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
    for epoch in range(2):
        hist, ctrl = run_epoch(rt, ctl, tokens, positions, gens, table)
        assert ctrl[3] == 0, f"epoch {epoch}: device status {ctrl[3]}"
        executed = ctrl[6 + 2 * B : 6 + 3 * B]
        assert all(e == 8 or ctrl[6 + 3 * B + r] == 1 for r, e in enumerate(executed))
        for r in range(B):
            if executed[r] > 0:
                tokens[r] = hist[executed[r] - 1, r]
                positions[r] += executed[r]
    key = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
    rt.read_state("key_cache", key)
    assert_close_rel(key.view_as(ctl.resident_key), ctl.resident_key, rel_tol(W.dims), "resident keys")
