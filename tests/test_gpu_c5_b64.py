"""GPU parity at the scaled batch: B=64 rows on one Qwen2.5-7B layer (bf16),
a 1024-block pool, 8 blocks of 128 per row, window 1024, contexts 256-1000.

Exercises the 8-row projection tiles (eight row tiles per projection), the
multi-tile attention (up to four 256-position tiles per row), the controller
at B=64 and random block tables from the pool.  The resident state of every
row is installed directly (seeded KV over the whole pool plus the rows'
generation/token/position), then one K=8 epoch runs on the device and in the
teacher-forced oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cruise_amd.runtime import pack_feed, tiling_bytes
from oracle.controller import EpochFeed, control_input_elements
from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C5, random_tables, slot_of
from parity import TeacherForcing, assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C5
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row


@pytest.fixture(scope="module")
def weights_pair():
    dev = generate_weights(W.dims, W.seed, device="cuda")
    cpu = {k: v.cpu() for k, v in dev.items()}
    return dev, cpu


@pytest.fixture(scope="module")
def rt(weights_pair):
    dev, _ = weights_pair
    r = make_runtime(W, dev)
    torch.cuda.synchronize()
    yield r
    r.close()


def test_b64_decoder_step(rt, weights_pair):
    _, cpu = weights_pair
    rng = np.random.default_rng(6400)
    table = random_tables(rng, B, BPR, W.geometry.physical_blocks)
    pos = rng.integers(256, 1000, size=B).astype(np.int64)
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = (rng.random(B) > 0.1).astype(np.int32)
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 670101, torch.bfloat16)
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
    written = [int(slot[r]) for r in range(B) if active[r]]
    mask = torch.ones(flat(key).shape[1], dtype=torch.bool)
    mask[written] = False
    for got, ref, inp, what in ((gk.cpu(), ref_k, key, "key"), (gv.cpu(), ref_v, value, "value")):
        assert torch.equal(flat(got)[:, mask], flat(inp)[:, mask]), f"unaddressed {what} slots changed"
        assert_close_rel(flat(got)[:, written], flat(ref)[:, written], rel_tol(W.dims), f"written {what}")


def test_b64_epoch_k8(rt, weights_pair):
    _, cpu = weights_pair
    rng = np.random.default_rng(6401)
    table = random_tables(rng, B, BPR, W.geometry.physical_blocks)
    pos = rng.integers(256, 1000, size=B).astype(np.int64)
    tok = rng.integers(0, W.dims.vocab, size=B).astype(np.int64)
    gens = np.arange(1, B + 1, dtype=np.int32)
    dec, ctl = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 670102, torch.bfloat16)
    # identical resident state on both sides
    rt.write_state("key_cache", key.cuda())
    rt.write_state("value_cache", value.cuda())
    rows = np.stack([gens, tok, pos, pos + 1, np.ones(B)]).astype(np.int64)
    rt.write_state("resident_rows", rows)
    ctl.resident_key, ctl.resident_value = key.clone(), value.clone()
    ctl.resident_generation = [int(g) for g in gens]
    ctl.resident_token = [int(t) for t in tok]
    ctl.resident_position = [int(p) for p in pos]
    ctl.resident_length = [int(p) + 1 for p in pos]
    ctl.resident_valid = [1] * B
    K = 8
    lengths = (pos + 1).astype(np.int32)
    active = np.ones(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[3 + B :] = gens
    slots = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    hist, ctrl = rt.proc(pack_feed(tok, pos, lengths, slots, active, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tok, pos, lengths, slots, active, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches, tf.mismatches[:5]
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    assert ctrl[3] == 0 and ctrl[4] == K
    for name, ref in (("key_cache", ctl.resident_key), ("value_cache", ctl.resident_value)):
        got = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
        rt.read_state(name, got)
        assert_close_rel(got.view_as(ref), ref, rel_tol(W.dims), f"resident {name}")
