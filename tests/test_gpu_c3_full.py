"""GPU parity at the full Qwen2.5-7B shape (28 layers, hidden 3584, 28/4
heads, head_dim 128, intermediate 18944, vocab 152064, bf16), B=4, block 128
x 2 blocks per row, capacity 256: the bench workload.

The engine generates its synthetic weights on the device; the oracle reads
the same bytes back.  Checked: one decoder step over a permuted block table
with seeded KV (logits, written KV, untouched KV, next positions), and two
consecutive K=8 epochs after prefilling 2-5 token prompts (history and control
record bit-exact with the teacher-forced oracle, resident caches at
tolerance), which exercises resident continuity across epochs at full size.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from cruise_amd.runtime import ResidentEpochRuntime, WeightSpec, pack_feed, tiling_bytes
from oracle.controller import EpochFeed, control_input_elements
from oracle.decoder import inv_freq, weight_shapes
from oracle.weights import seeded_cache
from oracle.workloads import C3, slot_of
from parity import TeacherForcing, assert_close_rel, engine_config, oracle_controller, rel_tol

pytestmark = pytest.mark.gpu

W = C3
B = W.geometry.batch
BS = W.geometry.block_size
BPR = W.geometry.blocks_per_row


@pytest.fixture(scope="module")
def rt_weights():
    rt = ResidentEpochRuntime(engine_config(W, weights=WeightSpec("synthetic", W.seed, 0.02)))
    rt.write_state("inv_freq", inv_freq(W.dims).contiguous())
    cpu = {}
    for name, shape in weight_shapes(W.dims).items():
        t = torch.empty(shape, dtype=torch.bfloat16)
        rt.read_state(name, t)
        cpu[name] = t
    yield rt, cpu
    rt.close()


def test_full_model_decoder_step(rt_weights):
    rt, cpu = rt_weights
    rng = np.random.default_rng(303)
    table = rng.permutation(B * BPR).astype(np.int32).reshape(B, BPR)
    ctx = np.array([2, 130, 57, 5], dtype=np.int64)  # row 1 crosses into its second block
    pos = ctx.copy()
    length = (pos + 1).astype(np.int32).reshape(B, 1)
    active = np.array([1, 1, 1, 1], dtype=np.int32)
    tok = rng.integers(0, W.dims.vocab, size=(B, 1)).astype(np.int64)
    slot = np.array([slot_of(table, r, int(pos[r]), BS) for r in range(B)], dtype=np.int32)
    dec, _ = oracle_controller(W, cpu)
    key, value = seeded_cache(dec.cache_shape(), 530041, torch.bfloat16)
    ref_logits, ref_k, ref_v, ref_next = dec.forward(
        torch.from_numpy(tok), torch.from_numpy(pos), torch.from_numpy(length), torch.from_numpy(table),
        torch.from_numpy(slot), key, value, None, torch.from_numpy(active),
    )
    gk, gv = key.clone().cuda(), value.clone().cuda()
    logits = torch.zeros(B, W.dims.vocab, dtype=torch.float32, device="cuda")
    nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
    rt.decoder_step(tok, pos, length, gk, slot, active, table, gv, logits, nxt)
    torch.cuda.synchronize()
    assert torch.equal(nxt.cpu(), ref_next)
    assert_close_rel(logits.cpu(), ref_logits.reshape(B, -1), rel_tol(W.dims), "logits")
    flat = lambda t: t.reshape(W.dims.num_layers, -1, W.dims.num_kv_heads, W.dims.head_dim)
    written = [int(s) for s in slot]
    mask = torch.ones(flat(key).shape[1], dtype=torch.bool)
    mask[written] = False
    for got, ref, inp, what in ((gk.cpu(), ref_k, key, "key"), (gv.cpu(), ref_v, value, "value")):
        assert torch.equal(flat(got)[:, mask], flat(inp)[:, mask]), f"unaddressed {what} slots changed"
        assert_close_rel(flat(got)[:, written], flat(ref)[:, written], rel_tol(W.dims), f"written {what}")
    for r in range(B):
        row = ref_logits[r, 0].numpy()
        top2 = np.sort(row)[-2:]
        if top2[1] - top2[0] > rel_tol(W.dims) * np.abs(row).max():
            assert int(logits[r].argmax()) == int(row.argmax())


def run_epoch(rt, ctl, tokens, positions, gens, table, K=8):
    lengths = (positions + 1).astype(np.int32)
    active = np.ones(B, dtype=np.int32)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = W.eos
    control[3 + B :] = gens
    slots = np.array([slot_of(table, r, int(positions[r]), BS) for r in range(B)], dtype=np.int32)
    hist, ctrl = rt.proc(pack_feed(tokens, positions, lengths, slots, active, table, tiling_bytes(), control))
    tf = TeacherForcing(hist, rel_tol(W.dims))
    ctl.token_override = tf
    ref = ctl.proc(EpochFeed(tokens, positions, lengths, slots, active, table.reshape(-1), tiling_bytes(), control))
    assert not tf.mismatches, tf.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    np.testing.assert_array_equal(ctrl, ref.control)
    return hist, ctrl


def test_full_model_two_epochs_after_prefill(rt_weights):
    rt, cpu = rt_weights
    rng = np.random.default_rng(W.seed)
    table = np.arange(B * BPR, dtype=np.int32).reshape(B, BPR)
    ps = [list(map(int, rng.integers(0, W.dims.vocab, size=int(rng.integers(2, 6))))) for _ in range(B)]
    _, ctl = oracle_controller(W, cpu)
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    gens = np.arange(1, B + 1, dtype=np.int32)
    for r in range(B):
        rt.prefill(r, int(gens[r]), ps[r], table[r])
        ctl.prefill_row(r, int(gens[r]), ps[r], table[r])
    tokens = np.array([p[-1] for p in ps], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
    for epoch in range(2):
        hist, ctrl = run_epoch(rt, ctl, tokens, positions, gens, table)
        assert ctrl[3] == 0, f"epoch {epoch}: device status {ctrl[3]}"
        executed = ctrl[6 + 2 * B : 6 + 3 * B]
        assert all(e == 8 or ctrl[6 + 3 * B + r] == 1 for r, e in enumerate(executed))
        for r in range(B):
            if executed[r] > 0:
                tokens[r] = hist[executed[r] - 1, r]
                positions[r] += executed[r]
    check_caches(rt, ctl)


def check_caches(rt, ctl):
    for name, ref in (("key_cache", ctl.resident_key), ("value_cache", ctl.resident_value)):
        got = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
        rt.read_state(name, got)
        assert_close_rel(got.view_as(ref), ref, rel_tol(W.dims), f"resident {name}")


def fresh_prefilled(rt, cpu, seed, table):
    rng = np.random.default_rng(seed)
    ps = [list(map(int, rng.integers(0, W.dims.vocab, size=int(rng.integers(2, 6))))) for _ in range(B)]
    _, ctl = oracle_controller(W, cpu)
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    gens = np.arange(1, B + 1, dtype=np.int32) + seed % 97
    for r in range(B):
        rt.prefill(r, int(gens[r]), ps[r], table[r])
        ctl.prefill_row(r, int(gens[r]), ps[r], table[r])
    tokens = np.array([p[-1] for p in ps], dtype=np.int64)
    positions = np.array([len(p) - 1 for p in ps], dtype=np.int64)
    return ctl, tokens, positions, gens


@pytest.mark.parametrize("K", [1, 2, 4])
def test_full_model_epoch_k(rt_weights, K):
    """One K-step epoch after prefilling, for each K of the sweep besides the
    bench's K=8 (each K runs its own captured graph)."""
    rt, cpu = rt_weights
    table = np.array([[3, 0], [6, 1], [2, 7], [5, 4]], dtype=np.int32)
    ctl, tokens, positions, gens = fresh_prefilled(rt, cpu, 3300 + K, table)
    print(f"[c3] K={K} epoch from positions {positions.tolist()}", flush=True)
    hist, ctrl = run_epoch(rt, ctl, tokens, positions, gens, table, K=K)
    assert ctrl[3] == 0 and ctrl[4] == K
    check_caches(rt, ctl)


def test_full_model_import_epoch_at_reference_payload(rt_weights):
    """A host-snapshot KV import at the reference's own geometry: 28 layers x 4
    rows x (K, V) x one 128-slot block of 4 x 128 bf16 = 29,360,128 bytes
    behind an 80-byte transfer header (native/resident_epoch_protocol.h:8-9,
    kv_transfer.py:31), through the bridge call, then a K=2 epoch.  Rows 0
    and 2 import a 3- and a 100-token prefix, row 1 starts a new generation,
    row 3 is empty."""
    import os
    import struct
    import tempfile
    import zlib

    from oracle.controller import IMPORT_GRAPH_FLAG

    rt, cpu = rt_weights
    L, KVH, D = W.dims.num_layers, W.dims.num_kv_heads, W.dims.head_dim
    block_elems = BS * KVH * D
    payload_t = (torch.randn(2 * L * B * block_elems, generator=torch.Generator().manual_seed(3307)) * 0.25).to(
        torch.bfloat16
    )
    payload = payload_t.view(torch.uint8).numpy().tobytes()
    assert len(payload) == 29_360_128
    mask = 0b0101
    gens = [7, 8, 9, 0]
    block_bytes = block_elems * 2
    checksum = 1
    for base in (0, L * B * block_bytes):  # kv_transfer.py:159-174 restated with zlib
        for layer in range(L):
            for row in range(B):
                if mask & (1 << row):
                    off = base + (layer * B + row) * block_bytes
                    checksum = zlib.adler32(payload[off : off + block_bytes], checksum)
    header = struct.pack("<QIIQQI4i7I", 0x4352554953454B56, 1, 80, 4242, len(payload), mask, *[7, 0, 9, 0],
                         L, B, BS, KVH, D, 2, checksum)
    tokens, positions, lengths = [17, 42, 99, 0], [3, 0, 100, 0], [4, 1, 101, 0]
    zeros = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16, device="cuda")
    rt.write_state("key_cache", zeros)
    rt.write_state("value_cache", zeros)
    rt.write_state("resident_rows", np.zeros((5, B), dtype=np.int64))
    fd, path = tempfile.mkstemp(prefix="cruise-kv7b-", dir="/dev/shm")
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(header)
            f.write(payload)
        out = rt.execute(3, 2, tokens, positions, lengths, [W.eos] * B, gens, transfer_path=path, transfer_id=4242)
    finally:
        os.unlink(path)
    assert out.status == 0 and out.device_status == 0, (out.status, out.device_status)
    assert out.kv_import_checksum == checksum & 0xFFFFFFFF
    assert out.declared_input_bytes == 29_360_128 + 260 - 16
    table = np.arange(B * BPR, dtype=np.int32).reshape(B, BPR)
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = 2
    control[1 : 1 + B] = W.eos
    control[2 + B] = IMPORT_GRAPH_FLAG | mask
    control[3 + B :] = gens
    _, ctl = oracle_controller(W, cpu)
    hist = np.full((8, B), -1, dtype=np.int64)
    for r in range(B):
        hist[: out.executed[r], r] = out.token_ids[r, : out.executed[r]]
    ctl.token_override = TeacherForcing(hist, rel_tol(W.dims))
    ref = ctl.proc(EpochFeed(np.array(tokens), np.array(positions), np.array(lengths, dtype=np.int32),
                             np.zeros(B, dtype=np.int32), np.array([1, 1, 1, 0], dtype=np.int32), table.reshape(-1),
                             tiling_bytes(), control, import_payload=payload))
    assert not ctl.token_override.mismatches, ctl.token_override.mismatches
    np.testing.assert_array_equal(hist, ref.history)
    assert int(np.uint32(np.int32(ref.control[5]))) == checksum & 0xFFFFFFFF
    np.testing.assert_array_equal(out.executed, ref.control[6 + 2 * B : 6 + 3 * B])
    check_caches(rt, ctl)
    # the imported prefixes are the payload, bit for bit
    key = torch.zeros(rt.cache_bytes // 2, dtype=torch.bfloat16)
    rt.read_state("key_cache", key)
    key = key.view(L, -1, BS, KVH, D)
    src = payload_t.view(2, L, B, BS, KVH, D)
    assert torch.equal(key[:, table[0, 0], :3].view(torch.int16), src[0, :, 0, :3].view(torch.int16))
    assert torch.equal(key[:, table[2, 0], :100].view(torch.int16), src[0, :, 2, :100].view(torch.int16))
