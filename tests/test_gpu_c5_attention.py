"""The grouped decode attention of the 64-row step (one Qwen2.5-7B-shape layer
in bf16, 28 query heads over 4 KV heads, window 1024) on the matrix cores --
in one workgroup per (row, KV head), the default, and split over the window
in 256-position tiles (`{"attention_split": 1}`) -- and on the vector units,
each against the oracle decoder at context lengths on
every tile edge: 1, 2, 255, 256, 257, 511, 512, 768, 1023 and 1024 positions
(a full window), plus random ones, with some rows inactive.

The versions round at the same points (the bf16 score, its bf16 scaling,
the bf16 probability, the bf16 output) and differ only in the order of fp32
sums, so both must meet the model tolerance against the oracle and the greedy
tokens must match it; the cache writes precede the attention and must be
identical.  A second case widens the window to 1280 positions (10 blocks per
row), so the matrix-core kernel requests its keys in two chunks of four
tiles.  The engine allows one instance per process, so the runtimes run one
after the other."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.decoder import PagedGeometry
from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C5, Workload, random_tables, slot_of
from parity import assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C5
# the same layer with 10 blocks of 128 per row: windows past four 256-position tiles
W1280 = Workload("qwen7b-1layer-b64-w1280", C5.dims,
                 PagedGeometry(batch=64, physical_blocks=1024, block_size=128, blocks_per_row=10, window=1280),
                 eos=C5.eos, seed=C5.seed)


@pytest.fixture(scope="module")
def weights_pair():
    dev = generate_weights(W.dims, W.seed, device="cuda")
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


def check_versions(w, weights_pair, edges, seed, cache_seed):
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
    key, value = seeded_cache(dec.cache_shape(), cache_seed, torch.bfloat16)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    inputs = (tok, pos, length, slot, active, table, key, value)
    tiles = (g.window + 255) // 256
    mode_m, got_m = run_step(w, dev, {}, inputs)
    mode_s, got_s = run_step(w, dev, {"attention_split": 1}, inputs)
    mode_v, got_v = run_step(w, dev, {"attention_mfma": 0}, inputs)
    assert mode_s == (2, tiles) and mode_m == (2, 0) and mode_v == (1, 0), (mode_s, mode_m, mode_v)
    for got, what in ((got_s, "matrix cores, split"), (got_m, "matrix cores"), (got_v, "vector units")):
        logits, nxt, gk, gv = got
        assert torch.equal(nxt, ref_next), what
        assert_close_rel(logits, ref_logits.reshape(B, -1), rel_tol(w.dims), f"logits ({what})")
    for got in (got_s, got_m):
        assert torch.equal(got[2], got_v[2]) and torch.equal(got[3], got_v[3])


def test_grouped_attention_versions_against_oracle(weights_pair):
    check_versions(W, weights_pair, (1, 2, 255, 256, 257, 511, 512, 768, 1023, 1024), 6403, 670104)


def test_grouped_attention_two_key_chunks_against_oracle(weights_pair):
    check_versions(W1280, weights_pair, (1, 256, 1023, 1024, 1025, 1100, 1279, 1280), 6404, 670105)
