"""Launch-plan variants of the 64-row matrix-core step (one Qwen2.5-7B-shape
layer in bf16): each must reproduce the default plan's logits, greedy tokens
and cache writes exactly.

- {"lm_cu": 0}: the LM head as 4-wave workgroups of two strips each with a
  separate argmax fold launch, instead of the default one workgroup per CU
  that stages the activations once in LDS and hands its per-CU argmax
  partials to the controller.  Every logit is the same chain of MFMA steps
  over k in the same order, so the two must agree bit for bit.
- {"mf_split": 0}: o and down as one workgroup per 16-column strip whose 8
  waves split K and add their sums in wave order, instead of the default
  split over (strip group, K range) with the 8 range partials added, in
  range order, by the next RMSNorm launch: the same sums in the same order.
- {"gu_cu": 0}: gate/up as 4-wave workgroups (each wave one strip of gate
  and up over the whole K) instead of one workgroup per CU whose waves run
  the same strips' step chains over LDS-staged activations.
- {"part_cu": 0}: the split o and down projections with every wave fetching
  its K range's activation fragments itself, instead of the workgroup staging
  them once in LDS: the same step chains (and qkv as in {"qkv_split": 0}).
- {"qkv_split": 0}: qkv as one workgroup per strip whose 8 waves split K and
  add their sums in wave order, instead of the split over (9-strip group, K
  range) whose 8 partials k_mf_qkv_finish adds in range order before the
  bias, RoPE and paged writes: the same sums in the same order.

The engine allows one instance per process, so the runtimes run one after
the other."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C5, random_tables, slot_of
from parity import make_runtime, oracle_controller

pytestmark = pytest.mark.gpu

W = C5
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row


@pytest.fixture(scope="module")
def weights_dev():
    return generate_weights(W.dims, W.seed, device="cuda")


def step_once(weights, tuning, inputs):
    tok, pos, length, slot, active, table, key, value = inputs
    rt = make_runtime(W, weights, tuning=tuning)
    try:
        facts = {k: rt.info(k) for k in ("lm_cu", "argmax_parts", "compute_units", "mf_split", "gu_cu", "part_cu", "qkv_split")}
        gk, gv = key.clone().cuda(), value.clone().cuda()
        logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
        torch.cuda.synchronize()
        return facts, (logits.cpu(), nxt.cpu(), gk.cpu(), gv.cpu())
    finally:
        rt.close()


@pytest.mark.parametrize(
    "tuning",
    [{"lm_cu": 0}, {"mf_split": 0}, {"gu_cu": 0}, {"part_cu": 0}, {"qkv_split": 0}],
    ids=["lm_cu0", "mf_split0", "gu_cu0", "part_cu0", "qkv_split0"],
)
def test_matrix_core_plan_variants_match_bit_for_bit(weights_dev, tuning):
    rng = np.random.default_rng(6402)
    table = random_tables(rng, B, BPR, W.geometry.physical_blocks)
    pos = rng.integers(256, 1000, size=B).astype(np.int64)
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = (rng.random(B) > 0.1).astype(np.int32)
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, {k: v.cpu() for k, v in weights_dev.items()})
    key, value = seeded_cache(dec.cache_shape(), 670103, torch.bfloat16)
    inputs = (tok, pos, length, slot, active, table, key, value)
    base_facts, base = step_once(weights_dev, {}, inputs)
    facts, got = step_once(weights_dev, tuning, inputs)
    assert base_facts["lm_cu"] == 1 and base_facts["argmax_parts"] == base_facts["compute_units"]
    assert base_facts["mf_split"] == 1 and base_facts["gu_cu"] == base_facts["compute_units"]
    assert base_facts["part_cu"] == 1 and base_facts["qkv_split"] == 1
    if "lm_cu" in tuning:
        assert facts["lm_cu"] == 0 and facts["argmax_parts"] == 1
    elif "mf_split" in tuning:
        assert facts["mf_split"] == 0 and facts["part_cu"] == 0 and facts["qkv_split"] == 0
    elif "part_cu" in tuning:
        assert facts["part_cu"] == 0 and facts["mf_split"] == 1 and facts["qkv_split"] == 0
    elif "qkv_split" in tuning:
        assert facts["qkv_split"] == 0 and facts["part_cu"] == 1
    else:
        assert facts["gu_cu"] == 0
    for name, a, b in zip(("logits", "next", "key", "value"), base, got):
        assert torch.equal(a, b), name
