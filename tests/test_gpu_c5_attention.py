"""The grouped decode attention of the 64-row step (one Qwen2.5-7B-shape layer
in bf16, 28 query heads over 4 KV heads, window 1024) on the matrix cores and
on the vector units, each against the oracle decoder at context lengths on
every tile edge: 1, 2, 255, 256, 257, 511, 512, 768, 1023 and 1024 positions
(a full window), plus random ones, with some rows inactive.

The two versions round at the same points (the bf16 score, its bf16 scaling,
the bf16 probability, the bf16 output) and differ only in the order of fp32
sums, so both must meet the model tolerance against the oracle and the greedy
tokens must match it; the cache writes precede the attention and must be
identical.  The engine allows one instance per process, so the runtimes run
one after the other."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C5, random_tables, slot_of
from parity import assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C5
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row
EDGES = (1, 2, 255, 256, 257, 511, 512, 768, 1023, 1024)


@pytest.fixture(scope="module")
def weights_pair():
    dev = generate_weights(W.dims, W.seed, device="cuda")
    return dev, {k: v.cpu() for k, v in dev.items()}


def run_step(weights, tuning, inputs):
    tok, pos, length, slot, active, table, key, value = inputs
    rt = make_runtime(W, weights, tuning=tuning)
    try:
        mode = rt.info("grouped_attention")
        gk, gv = key.clone().cuda(), value.clone().cuda()
        logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
        torch.cuda.synchronize()
        return mode, (logits.cpu(), nxt.cpu(), gk.cpu(), gv.cpu())
    finally:
        rt.close()


def test_grouped_attention_versions_against_oracle(weights_pair):
    dev, cpu = weights_pair
    rng = np.random.default_rng(6403)
    table = random_tables(rng, B, BPR, W.geometry.physical_blocks)
    ctx = rng.integers(1, BPR * BS + 1, size=B)
    ctx[: len(EDGES)] = EDGES
    pos = (ctx - 1).astype(np.int64)
    length = ctx.astype(np.int32).reshape(B, 1)
    active = (rng.random(B) > 0.15).astype(np.int32)
    active[: len(EDGES)] = 1
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 670104, torch.bfloat16)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    inputs = (tok, pos, length, slot, active, table, key, value)
    mode_m, got_m = run_step(dev, {}, inputs)
    mode_v, got_v = run_step(dev, {"attention_mfma": 0}, inputs)
    assert mode_m == 2 and mode_v == 1
    for got, what in ((got_m, "matrix cores"), (got_v, "vector units")):
        logits, nxt, gk, gv = got
        assert torch.equal(nxt, ref_next), what
        assert_close_rel(logits, ref_logits.reshape(B, -1), rel_tol(W.dims), f"logits ({what})")
    assert torch.equal(got_m[2], got_v[2]) and torch.equal(got_m[3], got_v[3])
