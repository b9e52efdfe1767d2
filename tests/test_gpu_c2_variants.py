"""Launch-plan variants on one Qwen2.5-7B-shape bf16 layer: each must give
exactly the default plan's logits, greedy tokens and cache writes.

- {"o_waves": 4}: 448 4-wave o-projection workgroups against the default
  one 7-wave workgroup per 7 row pairs (one per CU on a 256-CU MI355X); the
  per-pair code is the same, so the results must be too.

Both sides also run the row-pair qkv kernel ({"qkv_ksplit": 0}), so the
comparison covers it next to the default K-split qkv, whose sums run in
another fp32 order and are checked against the oracle by the layer tests.

The engine allows one instance per process, so the runtimes run one after
the other."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C2, random_tables, slot_of
from parity import make_runtime, oracle_controller

pytestmark = pytest.mark.gpu

W = C2
B = W.geometry.batch
BS = W.geometry.block_size


@pytest.fixture(scope="module")
def weights_dev():
    return generate_weights(W.dims, W.seed, device="cuda")


def step_once(weights, tuning, inputs):
    tok, pos, length, slot, active, table, key, value = inputs
    rt = make_runtime(W, weights, tuning=tuning)
    try:
        facts = {k: rt.info(k) for k in ("o_waves", "o_grid", "compute_units", "qkv_ksplit")}
        gk, gv = key.clone().cuda(), value.clone().cuda()
        logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
        torch.cuda.synchronize()
        return facts, (logits.cpu(), nxt.cpu(), gk.cpu(), gv.cpu())
    finally:
        rt.close()


@pytest.mark.parametrize("tuning", [{"o_waves": 4}], ids=["o4"])
def test_projection_workgroup_shapes_match_bit_for_bit(weights_dev, tuning):
    rng = np.random.default_rng(77)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    pos = rng.integers(2, 6, size=B).astype(np.int64)
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = np.array([1, 1, 0, 1], dtype=np.int32)
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, {k: v.cpu() for k, v in weights_dev.items()})
    key, value = seeded_cache(dec.cache_shape(), 5150, torch.bfloat16)
    inputs = (tok, pos, length, slot, active, table, key, value)
    base_facts, base = step_once(weights_dev, {"qkv_ksplit": 0}, inputs)
    facts, got = step_once(weights_dev, {"qkv_ksplit": 0, **tuning}, inputs)
    cus = base_facts["compute_units"]
    o_pairs = W.dims.hidden // 2
    if o_pairs == 7 * cus:
        assert base_facts["o_waves"] == 7 and base_facts["o_grid"] == cus
    assert base_facts["qkv_ksplit"] == 0 and facts["qkv_ksplit"] == 0
    if "o_waves" in tuning:
        assert facts["o_waves"] == 4 and facts["o_grid"] == (o_pairs + 3) // 4
    for name, a, b in zip(("logits", "next", "key", "value"), base, got):
        assert torch.equal(a, b), name
