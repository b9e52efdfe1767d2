"""The persistent step kernel against the per-op launches.

Both paths compute every output with the same dot order, wave reductions,
rounding points and segment order, so on the same inputs they must agree bit
for bit: decoder-step logits, written and untouched KV, and, over several
consecutive K=8 epochs after prefilling 2-5 token prompts, the epoch
histories, control records and the resident caches.  A difference in any bit
means a hand-off between workgroups of the persistent kernel read a value
before it was written (or a stale copy).  The per-op path (the default) is
checked against the oracle by the C1-C5 tests; here it is the reference.

Workloads: one Qwen2.5-7B layer (C2 shape, block table permuted over a
64-block pool) and the full 28-layer model (the bench workload), plus an
epoch that starts from an empty row and one with an inactive row.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest
import torch

from cruise_amd.runtime import ResidentEpochRuntime, WeightSpec, pack_feed, tiling_bytes
from oracle.controller import control_input_elements
from oracle.decoder import inv_freq
from oracle.weights import seeded_cache
from oracle.workloads import C2, C3, slot_of
from parity import engine_config

pytestmark = pytest.mark.gpu


def make_engine(w, fused: bool, capacity: int) -> ResidentEpochRuntime:
    cfg = engine_config(w, capacity=capacity, weights=WeightSpec("synthetic", w.seed, 0.02))
    cfg = replace(cfg, engine=replace(cfg.engine, fused_step=fused))
    rt = ResidentEpochRuntime(cfg)
    rt.write_state("inv_freq", inv_freq(w.dims).contiguous())
    assert rt.info("fused_step") == (1 if fused else 0)
    return rt


def run_workload(w, fused: bool, epochs: int, capacity: int) -> dict:
    """Decoder step over seeded KV, then prefill + `epochs` K=8 epochs."""
    g = w.geometry
    B, BS, BPR = g.batch, g.block_size, g.blocks_per_row
    rt = make_engine(w, fused, capacity)
    out = {}
    try:
        rng = np.random.default_rng(4242)
        table = rng.permutation(g.physical_blocks)[: B * BPR].astype(np.int32).reshape(B, BPR)
        # decoder-step ABI: permuted blocks, contexts in both blocks, one inactive row
        pos = np.array([2, min(130, capacity - 2), 57, 5], dtype=np.int64)[:B]
        length = (pos + 1).astype(np.int32).reshape(B, 1)
        active = np.array([1, 1, 0, 1], dtype=np.int32)[:B]
        tok = rng.integers(0, w.dims.vocab, size=(B, 1)).astype(np.int64)
        slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
        shape = (w.dims.num_layers, g.physical_blocks, BS, w.dims.num_kv_heads, w.dims.head_dim)
        key, value = seeded_cache(shape, 530041, torch.bfloat16)
        gk, gv = key.clone().cuda(), value.clone().cuda()
        logits = torch.zeros(B, w.dims.vocab, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
        torch.cuda.synchronize()
        out["step_logits"] = logits.cpu()
        out["step_key"] = gk.cpu()
        out["step_value"] = gv.cpu()
        out["step_next"] = nxt.cpu()

        # resident epochs from prefilled prompts
        zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
        rt.write_state("key_cache", zeros)
        rt.write_state("value_cache", zeros)
        rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
        prng = np.random.default_rng(w.seed)
        ps = [list(map(int, prng.integers(0, w.dims.vocab, size=int(prng.integers(2, 6))))) for _ in range(B)]
        gens = np.arange(1, B + 1, dtype=np.int32)
        for r in range(B):
            rt.prefill(r, int(gens[r]), ps[r], table[r])
        tokens = np.array([p[-1] for p in ps], dtype=np.int64)
        positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
        hists, ctrls = [], []
        for _ in range(epochs):
            lengths = (positions + 1).astype(np.int32)
            act = np.ones(B, dtype=np.int32)
            control = np.zeros(control_input_elements(B), dtype=np.int32)
            control[0] = 8
            control[1 : 1 + B] = -1 if w.eos is None else w.eos
            control[3 + B :] = gens
            slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
            hist, ctrl = rt.proc(pack_feed(tokens, positions, lengths, slots, act, table, tiling_bytes(), control))
            hists.append(hist.copy())
            ctrls.append(ctrl.copy())
            if ctrl[3] != 0:
                break
            executed = ctrl[6 + 2 * B : 6 + 3 * B]
            if int(executed.min()) < 8:
                break  # a row hit EOS; both paths stop here
            for r in range(B):
                tokens[r] = hist[executed[r] - 1, r]
                positions[r] += executed[r]
            if int(positions.max()) + 8 >= capacity:
                break
        out["hist"] = hists
        out["ctrl"] = ctrls
        kc = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
        vc = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
        rt.read_state("key_cache", kc)
        rt.read_state("value_cache", vc)
        out["key"] = kc
        out["value"] = vc
    finally:
        rt.close()
    return out


def assert_same(a: dict, b: dict) -> None:
    for name in ("step_logits", "step_key", "step_value", "step_next", "key", "value"):
        x, y = a[name], b[name]
        if not torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x,
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y):
            diff = (x.float() - y.float()).abs()
            raise AssertionError(f"{name}: {int((diff != 0).sum())} elements differ, max |diff| {float(diff.max())}")
    assert len(a["hist"]) == len(b["hist"])
    for e, (h0, h1, c0, c1) in enumerate(zip(a["hist"], b["hist"], a["ctrl"], b["ctrl"])):
        np.testing.assert_array_equal(h1, h0, err_msg=f"epoch {e} history")
        np.testing.assert_array_equal(c1, c0, err_msg=f"epoch {e} control record")


@pytest.mark.parametrize("w,epochs,capacity", [(C2, 3, 256), (C3, 6, 256)], ids=["one_layer", "full_model"])
def test_persistent_kernel_matches_per_op_path(w, epochs, capacity):
    print(f"[fused] {w.name}: per-op path", flush=True)
    ref = run_workload(w, False, epochs, capacity)
    print(f"[fused] {w.name}: persistent kernel", flush=True)
    got = run_workload(w, True, epochs, capacity)
    assert all(c[3] == 0 for c in ref["ctrl"]), [int(c[3]) for c in ref["ctrl"]]
    print(f"[fused] {w.name}: {len(ref['ctrl'])} epochs compared", flush=True)
    assert len(ref["ctrl"]) >= 2
    assert_same(ref, got)


def test_persistent_kernel_is_deterministic():
    """Two runs of the persistent kernel on the same inputs agree bit for bit
    (a hand-off that sometimes reads early would show up as a difference)."""
    a = run_workload(C3, True, 2, 256)
    b = run_workload(C3, True, 2, 256)
    assert_same(a, b)
