"""GPU parity on one Qwen2.5-7B-shape layer in bf16 (hidden 3584, 28/4 heads,
head_dim 128, intermediate 18944, vocab 152064) over a 64-block pool with
random block tables: the decoder step's logits, slot writes and attention
against the oracle, and an epoch with a 7-position continuation."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.controller import EpochFeed, control_input_elements
from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C2, random_tables, slot_of
from cruise_amd.runtime import pack_feed, tiling_bytes
from parity import TeacherForcing, assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C2
B = W.geometry.batch
BS = W.geometry.block_size


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


@pytest.mark.parametrize("seed", [0, 1])
def test_decoder_step_random_tables(rt, weights_pair, seed):
    _, cpu = weights_pair
    rng = np.random.default_rng(1000 + seed)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    ctx = rng.integers(2, 6, size=B)  # existing context lengths 2-5
    pos = ctx.astype(np.int64)  # the new token sits at position ctx
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = np.array([1, 1, 1, 1], dtype=np.int32)
    if seed == 1:
        active[2] = 0  # an inactive row writes nothing
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 530041 + seed, torch.bfloat16)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    gk = key.clone().cuda()
    gv = value.clone().cuda()
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
    # greedy tokens agree wherever the margin is decisive
    for r in range(B):
        row = ref_logits[r, 0].numpy()
        top2 = np.sort(row)[-2:]
        if top2[1] - top2[0] > rel_tol(W.dims) * np.abs(row).max():
            assert int(logits[r].argmax()) == int(row.argmax())


@pytest.mark.parametrize("K", [1, 2, 4, 8])
def test_epoch_random_tables(rt, weights_pair, K):
    """Prefill 2-5 token prompts into random blocks, then one K-step epoch
    (every K of the resident epoch: each runs its own captured graph)."""
    _, cpu = weights_pair
    rng = np.random.default_rng(77 + K)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    ps = [list(map(int, rng.integers(0, W.dims.vocab, size=int(rng.integers(2, 6))))) for _ in range(B)]
    dec, ctl = oracle_controller(W, cpu)
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    for r in range(B):
        rt.prefill(r, 10 + r, ps[r], table[r])
        ctl.prefill_row(r, 10 + r, ps[r], table[r])
    tokens = np.array([p[-1] for p in ps], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
    lengths = (positions + 1).astype(np.int32)
    active = np.ones(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[3 + B : 3 + 2 * B] = 10 + np.arange(B)
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    hist, ctrl_out = rt.proc(pack_feed(tokens, positions, lengths, slots, active, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches, tf.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl_out, ref.control)
    assert ctrl_out[3] == 0 and ctrl_out[4] == K
    gk = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
    rt.read_state("key_cache", gk)
    assert_close_rel(gk.view_as(ctl.resident_key), ctl.resident_key, rel_tol(W.dims), "resident keys")
