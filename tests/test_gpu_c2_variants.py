"""The two qkv kernels on one Qwen2.5-7B-shape bf16 layer: the default K-split
qkv (k_qkv_ksplit: one 7-wave workgroup per CU, K split over the waves) and
the row-pair kernel every other shape runs ({"qkv_ksplit": 0}: one RoPE row
pair per wave over the whole K).  Their fp32 sums run in different orders, so
each is held to the oracle: logits within the model tolerance, the greedy
tokens exact, the written K/V slots within the tolerance and every other
slot untouched.

The engine allows one instance per process, so the runtimes run one after
the other."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.weights import generate_weights, seeded_cache
from oracle.workloads import C2, random_tables, slot_of
from parity import assert_close_rel, make_runtime, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C2
B = W.geometry.batch
BS = W.geometry.block_size


@pytest.fixture(scope="module")
def weights_pair():
    dev = generate_weights(W.dims, W.seed, device="cuda")
    return dev, {k: v.cpu() for k, v in dev.items()}


def step_once(weights, tuning, inputs):
    tok, pos, length, slot, active, table, key, value = inputs
    rt = make_runtime(W, weights, tuning=tuning)
    try:
        ksplit = rt.info("qkv_ksplit")
        gk, gv = key.clone().cuda(), value.clone().cuda()
        logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
        torch.cuda.synchronize()
        return ksplit, (logits.cpu(), nxt.cpu(), gk.cpu(), gv.cpu())
    finally:
        rt.close()


def test_qkv_kernels_against_oracle(weights_pair):
    dev, cpu = weights_pair
    rng = np.random.default_rng(77)
    table = random_tables(rng, B, W.geometry.blocks_per_row, W.geometry.physical_blocks)
    pos = rng.integers(2, 6, size=B).astype(np.int64)
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = np.array([1, 1, 0, 1], dtype=np.int32)
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 5150, torch.bfloat16)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    inputs = (tok, pos, length, slot, active, table, key, value)
    flat = lambda t: t.reshape(W.dims.num_layers, -1, W.dims.num_kv_heads, W.dims.head_dim)
    written = [int(slot[r]) for r in range(B) if active[r]]
    mask = torch.ones(flat(key).shape[1], dtype=torch.bool)
    mask[written] = False
    modes = []
    for tuning in ({}, {"qkv_ksplit": 0}):
        ksplit, (logits, nxt, gk, gv) = step_once(dev, tuning, inputs)
        modes.append(ksplit)
        what = f"qkv_ksplit={ksplit}"
        assert torch.equal(nxt, ref_next), what
        assert_close_rel(logits, ref_logits.reshape(B, -1), rel_tol(W.dims), f"logits ({what})")
        for got, ref, inp, name in ((gk, ref_k, key, "key"), (gv, ref_v, value, "value")):
            assert torch.equal(flat(got)[:, mask], flat(inp)[:, mask]), f"unaddressed {name} slots changed ({what})"
            assert_close_rel(flat(got)[:, written], flat(ref)[:, written], rel_tol(W.dims), f"written {name} ({what})")
    assert modes[0] > 0 and modes[1] == 0, modes
