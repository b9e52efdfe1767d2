"""Decode attention over long windows at few rows: one Qwen2.5-7B-shape layer
in bf16 (28 query heads over 4 KV heads) with 12 rows and a 4,096-position
window (32 blocks of 128 per row), so the per-(row, head) attention runs,
split over the window in 16 tiles of 256 positions (the default past 768
positions) and serially (`{"attention_split": 0}`), each against the oracle
decoder.  Contexts sit on the tile and block edges up to a full window:
1, 255, 256, 257, 2047, 2048, 2049, 3000, 4095 and 4096 positions, plus
random ones, with some rows inactive.

The two versions round at the same points (the bf16 score and its bf16
scaling, the probability rounded to bf16 after the row's exact max and sum,
the bf16 output) and differ only in the order of fp32 sums, so both must
meet the model tolerance against the oracle and the greedy tokens must match
it; the first layer's cache writes precede the attention and must be
identical, and every layer's must meet the tolerance against the oracle.  A second
case forces the split on a 512-position window, where the default walks the
tiles serially.  A third runs 16 rows (64 (row, KV head) pairs) at the
4,096-position window, past the LDS of the single-launch grouped kernels:
the matrix-core grouped attention split over the window is the default
there, checked against the oracle and against the per-head split
(`{"grouped_attention": 0}`).  A fourth runs the tiny fp32 model (head_dim
64, blocks of 16 positions) at a 1,024-position window, split by default,
against the serial tiles.  The engine allows one instance per process,
so the runtimes run one after the other."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.decoder import PagedGeometry
from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C1, C2, Workload, random_tables, slot_of
from parity import assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W4096 = Workload("qwen7b-1layer-b12-w4096", C2.dims,
                 PagedGeometry(batch=12, physical_blocks=512, block_size=128, blocks_per_row=32, window=4096),
                 eos=C2.eos, seed=C2.seed)
W4096_B16 = Workload("qwen7b-1layer-b16-w4096", C2.dims,
                     PagedGeometry(batch=16, physical_blocks=640, block_size=128, blocks_per_row=32, window=4096),
                     eos=C2.eos, seed=C2.seed)
# the tiny fp32 model (head_dim 64) with 64 blocks of 16 positions per row
W1024_FP32 = Workload("tiny-fp32-w1024", C1.dims,
                      PagedGeometry(batch=4, physical_blocks=256, block_size=16, blocks_per_row=64, window=1024),
                      eos=C1.eos, seed=C1.seed)
W512 = Workload("qwen7b-1layer-b12-w512", C2.dims,
                PagedGeometry(batch=12, physical_blocks=64, block_size=128, blocks_per_row=4, window=512),
                eos=C2.eos, seed=C2.seed)


@pytest.fixture(scope="module")
def weights_pair():
    dev = generate_weights(C2.dims, C2.seed, device="cuda")
    return dev, {k: v.cpu() for k, v in dev.items()}


def run_step(w, weights, tuning, inputs):
    tok, pos, length, slot, active, table, key, value = inputs
    B = w.geometry.batch
    rt = make_runtime(w, weights, tuning=tuning)
    try:
        mode = (rt.info("grouped_attention"), rt.info("attention_split"))
        gk, gv = key.clone().cuda(), value.clone().cuda()
        logits = torch.zeros(B, w.dims.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
        torch.cuda.synchronize()
        return mode, (logits.cpu(), nxt.cpu(), gk.cpu(), gv.cpu())
    finally:
        rt.close()


def check_split(w, weights_pair, edges, seed, cache_seed, split_tuning, serial_tuning, tiles,
                modes=None):
    dev, cpu = weights_pair
    g = w.geometry
    B, BS, BPR = g.batch, g.block_size, g.blocks_per_row
    rng = np.random.default_rng(seed)
    table = random_tables(rng, B, BPR, g.physical_blocks)
    ctx = rng.integers(1, g.window + 1, size=B)
    ctx[: len(edges)] = edges
    pos = (ctx - 1).astype(np.int64)
    length = ctx.astype(np.int32).reshape(B, 1)
    active = (rng.random(B) > 0.15).astype(np.int32)
    active[: len(edges)] = 1
    tok = rng.integers(0, w.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(w, cpu)
    cache_dtype = torch.float32 if w.dims.dtype == "fp32" else torch.bfloat16
    key, value = seeded_cache(dec.cache_shape(), cache_seed, cache_dtype)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    inputs = (tok, pos, length, slot, active, table, key, value)
    mode_s, got_s = run_step(w, dev, split_tuning, inputs)
    mode_t, got_t = run_step(w, dev, serial_tuning, inputs)
    want = modes if modes is not None else ((0, tiles), (0, 0))
    assert (mode_s, mode_t) == want, (mode_s, mode_t)
    for got, what in ((got_s, f"{split_tuning} {mode_s}"), (got_t, f"{serial_tuning} {mode_t}")):
        logits, nxt, gk, gv = got
        assert torch.equal(nxt, ref_next), what
        assert_close_rel(logits, ref_logits.reshape(B, -1), rel_tol(w.dims), f"logits ({what})")
    # layer 0's cache writes precede any attention: identical; later layers'
    # follow the previous attention's output: within the tolerance of the oracle
    layers = w.dims.num_layers
    for i, ref in ((2, ref_k), (3, ref_v)):
        assert torch.equal(got_s[i].reshape(layers, -1)[0], got_t[i].reshape(layers, -1)[0])
        for got in (got_s, got_t):
            assert_close_rel(got[i], ref.reshape(got[i].shape), rel_tol(w.dims), "cache")


def test_window_split_4096_against_oracle(weights_pair):
    check_split(W4096, weights_pair, (1, 255, 256, 257, 2047, 2048, 2049, 3000, 4095, 4096), 7401, 770101,
                {}, {"attention_split": 0}, 16)


def test_window_split_forced_512_against_oracle(weights_pair):
    check_split(W512, weights_pair, (1, 2, 255, 256, 257, 300, 511, 512), 7402, 770102,
                {"attention_split": 1}, {}, 2)


def test_grouped_split_4096_against_oracle(weights_pair):
    check_split(W4096_B16, weights_pair, (1, 255, 256, 257, 1024, 2047, 2049, 3000, 4095, 4096), 7403, 770103,
                {}, {"grouped_attention": 0}, 16, modes=((2, 16), (0, 16)))


def test_window_split_fp32_1024_against_oracle():
    dev = generate_weights(C1.dims, C1.seed, device="cuda")
    pair = (dev, {k: v.cpu() for k, v in dev.items()})
    check_split(W1024_FP32, pair, (1, 256, 1023, 1024), 7404, 770104, {}, {"attention_split": 0}, 4)
