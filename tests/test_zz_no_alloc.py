"""resident_epoch_prefill_batch_noalloc against resident_epoch_prefill_batch,
both through the C-ABI, on the same inputs from the same zeroed state: the
resident caches bit for bit and the resident rows exactly, for two calls in a
row of which the second is smaller (the fixed scratch keeps the first call's
contents).  Both paths run the same hand-written kernels, so they compute
the same values in the same order.  Also: device memory does not grow across a no-allocation call, and a
pass larger than the fixed scratch is refused (-3) before anything runs.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.weights import generate_weights
from oracle.workloads import C1, C2, random_tables
from parity import engine_snapshot, make_runtime

pytestmark = pytest.mark.gpu


def reset(rt, dtype, B):
    elems = rt.cache_bytes // torch.tensor([], dtype=dtype).element_size()
    zeros = torch.zeros(elems, dtype=dtype, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))


def same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    view = torch.int16 if a.dtype == torch.bfloat16 else torch.int32
    return torch.equal(a.view(view), b.view(view))


def compare_calls(W, rt, calls, check_memory=False):
    B = W.geometry.batch
    dtype = W.dims.torch_dtype
    for lengths, seed in calls:
        rng = np.random.default_rng(seed)
        n = len(lengths)
        table = random_tables(rng, n, W.geometry.blocks_per_row, W.geometry.physical_blocks)
        rows = sorted(rng.choice(B, size=n, replace=False).tolist())
        gens = [100 + seed % 50 + i for i in range(n)]
        prompts = [list(map(int, rng.integers(0, W.dims.vocab, size=m))) for m in lengths]
        print(f"[noalloc] {W.name}: rows {rows} prompt lengths {lengths}", flush=True)
        reset(rt, dtype, B)
        rt.prefill_batch(rows, gens, prompts, table)
        k_ref, v_ref, rows_ref = engine_snapshot(rt, dtype)
        reset(rt, dtype, B)
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        rt.prefill_batch(rows, gens, prompts, table, noalloc=True)
        torch.cuda.synchronize()
        free_after = torch.cuda.mem_get_info()[0]
        k, v, rows_got = engine_snapshot(rt, dtype)
        assert same_bits(k, k_ref), "keys differ from resident_epoch_prefill_batch"
        assert same_bits(v, v_ref), "values differ from resident_epoch_prefill_batch"
        np.testing.assert_array_equal(rows_got, rows_ref)
        if check_memory:
            # the grown-on-demand scratch of this pass would take M x ~69 KB
            assert free_before - free_after < (4 << 20), (free_before, free_after)


def test_noalloc_prefill_matches_tiny_fp32():
    w = generate_weights(C1.dims, C1.seed)
    rt = make_runtime(C1, w)
    try:
        compare_calls(C1, rt, [([29, 7, 20, 1], 7101), ([5, 3], 7102)])
    finally:
        rt.close()


def test_noalloc_prefill_matches_bf16_layer_and_refuses_oversize():
    dev = generate_weights(C2.dims, C2.seed, device="cuda")
    rt = make_runtime(C2, dev)
    try:
        compare_calls(C2, rt, [([70, 41, 5, 1], 7103), ([12, 2], 7104)], check_memory=True)
        # 4 x 250 tokens need ~66 MiB of scratch (more than the 64 MiB array): refused before any launch
        rng = np.random.default_rng(7105)
        prompts = [list(map(int, rng.integers(0, C2.dims.vocab, size=250))) for _ in range(4)]
        table = random_tables(rng, 4, C2.geometry.blocks_per_row, C2.geometry.physical_blocks)
        with pytest.raises(RuntimeError, match="-3"):
            rt.prefill_batch([0, 1, 2, 3], [1, 2, 3, 4], prompts, table, noalloc=True)
    finally:
        rt.close()
