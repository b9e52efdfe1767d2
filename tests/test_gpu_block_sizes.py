"""GPU parity of the decoder step at a block size that is not a power of two.

The decode attention computes a position's block and offset within the
block by shift and mask when the block size is a power of two, and by
division otherwise; every other workload here uses 16 or 128.  This runs the
tiny fp32 model (2 layers, hidden 256, 4/2 heads, head_dim 64) with blocks of
12 positions, 3 per row, a permuted block table, and positions at and around
block boundaries, against the oracle (the gather of position p from slot
table[b][p // bs] * bs + p % bs, batched_decoder_step.py:266-273)."""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle.decoder import PagedGeometry
from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C1, slot_of
from parity import assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = replace(C1, name="tiny-fp32-block12",
            geometry=PagedGeometry(batch=4, physical_blocks=12, block_size=12, blocks_per_row=3, window=36))
B = W.geometry.batch
BS = W.geometry.block_size
TABLE = np.asarray([[2, 7, 0], [5, 1, 9], [11, 3, 6], [4, 10, 8]], dtype=np.int32)
CASES = {
    "spread": [0, 13, 25, 35],          # first position, into block 2, block 3, last of the window
    "boundaries": [11, 12, 23, 24],     # last of a block, first of the next
}


@pytest.fixture(scope="module")
def weights():
    return generate_weights(W.dims, W.seed)


@pytest.fixture(scope="module")
def rt(weights):
    r = make_runtime(W, weights)
    yield r
    r.close()


@pytest.mark.parametrize("case", sorted(CASES))
def test_decoder_step_block12_matches_oracle(rt, weights, case):
    seed = 671200 + sorted(CASES).index(case)
    rng = np.random.default_rng(seed)
    pos = np.asarray(CASES[case], dtype=np.int64)
    tok64 = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    len32 = (pos + 1).astype(np.int32).reshape(B, 1)
    act32 = np.ones(B, dtype=np.int32)
    slot = np.array([slot_of(TABLE, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, weights)
    key, value = seeded_cache(dec.cache_shape(), seed, torch.float32)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok64), torch.from_numpy(pos), torch.from_numpy(len32), torch.from_numpy(TABLE),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(act32),
    )
    gk, gv = key.clone(), value.clone()
    logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32)
    nxt = torch.zeros(B, dtype=torch.int64)
    rt.decoder_step(tok64, pos, len32, gk, slot, act32, TABLE, gv, logits, nxt)
    assert torch.equal(nxt, ref_next), case
    assert_close_rel(logits, ref_logits.reshape(B, -1), rel_tol(W.dims), f"{case} logits")
    flat = (W.dims.num_layers, -1, W.dims.num_kv_heads, W.dims.head_dim)
    written = [int(s) for s in slot]
    mask = torch.ones(key.reshape(flat).shape[1], dtype=torch.bool)
    mask[written] = False
    for name, got, ref, before in (("keys", gk, ref_k, key), ("values", gv, ref_v, value)):
        assert torch.equal(got.reshape(flat)[:, mask], before.reshape(flat)[:, mask]), f"{case}: other {name} changed"
        assert_close_rel(got.reshape(flat)[:, written], ref.reshape(flat)[:, written], rel_tol(W.dims),
                         f"{case} written {name}")
