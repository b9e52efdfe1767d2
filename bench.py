#!/usr/bin/env python3
"""Resident decode epoch benchmark on one MI355X.

Workload: Qwen2.5-7B-shape decoder (28 layers, hidden 3584, GQA 28/4,
head_dim 128, intermediate 18944, vocab 152064, untied LM head), random-init
bf16 weights N(0, 0.02) generated on the device, B=4 rows, block size 128
with 2 blocks per row, greedy epochs of K=8 decoder steps through the
library's bridge call ``resident_epoch_execute`` (one host-to-device feed,
one device-to-host fetch per epoch).

A benchmark "step" is one K=8 epoch.  ``value`` is decoded tokens per second
(sum of executed steps over all rows / wall time of the timed epochs, inputs
resident in HBM; each epoch is one graph launch).

``roofline`` reports the dominant kernel, the gate/up projection (54% of the
streamed bytes).  Its launch duration is the mean over the 28 layers' gate/up
launched one after another between two HIP events on the engine's stream
(``--kernel-passes`` passes): each launch streams another layer's 272 MB, so
no launch finds its weights in the 256 MB memory-side cache, as in the epoch
graph.  The same launch timed inside ``--kernel-epochs`` epochs (events
around the middle layer's gate/up of the last step) is reported beside it;
it carries the events' own overhead.  ``cpu_baseline`` times the oracle's CPU
decoder path on the host cores over K=8 epochs of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

METRIC = "Qwen2.5-7B B=4 K=8 epoch decode tok/s; % of HBM weight-stream roofline"
HBM_PEAK_GBS = 8000.0
EOS = 151645


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20, help="timed K=8 epochs")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--epoch-steps", type=int, default=8)
    p.add_argument("--seed", type=int, default=20263)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-epochs", type=int, default=5, help="timed K=8 epochs of the CPU baseline")
    p.add_argument("--kernel-epochs", type=int, default=10)
    p.add_argument("--kernel-passes", type=int, default=4, help="passes over the 28 layers' gate/up launches")
    p.add_argument("--sweep-epochs", type=int, default=20,
                   help="timed epochs at each of K=1, 2, 4 (the K sweep beside the K=8 headline; 0 skips it)")
    p.add_argument("--tuning", default="", help="JSON object of launch-plan overrides (an A/B switch; the "
                                                 "headline uses the default plan)")
    p.add_argument("--workload", choices=("qwen7b-b4", "scaled-b64"), default="qwen7b-b4",
                   help="qwen7b-b4: the headline line; scaled-b64: one Qwen2.5-7B layer at 64 rows, contexts "
                        "256-1016, K=8 (a separate line, not the headline)")
    return p.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    args = parse_args()
    world = int(os.getenv("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(
            json.dumps({"error": "this build measures one GPU only; run with --gpus 1 (no multi-GPU path is built)"}),
            flush=True,
        )
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from cruise_amd.runtime import EngineConfig, EngineSpec, ModelSpec, ResidentEpochRuntime, WeightSpec

    if args.workload == "scaled-b64":
        return bench_scaled(args)
    K = args.epoch_steps
    cfg = EngineConfig(
        model=ModelSpec(),
        engine=EngineSpec(
            batch=4, physical_blocks=8, block_size=128, blocks_per_row=2, logical_capacity=256
        ),
        weights=WeightSpec(source="synthetic", seed=args.seed, std=0.02),
        tuning=json.loads(args.tuning) if args.tuning else {},
    )
    t0 = time.time()
    rt = ResidentEpochRuntime(cfg)
    B = rt.batch
    log(f"engine up in {time.time() - t0:.1f}s: {rt.info('streamed_weight_bytes') / 1e9:.3f} GB streamed per step")
    capacity = rt.info("capacity")
    rng = np.random.default_rng(args.seed)
    vocab = rt.vocab

    # Per-row generation state.  Rows start with a 2-5 token prompt (prefilled),
    # continue epoch after epoch, and restart with a new generation when the
    # next epoch would pass the capacity or the row emitted EOS.
    gens = [0] * B
    next_gen = [1]
    tokens = [0] * B
    positions = [0] * B

    def start_row(r: int) -> None:
        prompt = list(map(int, rng.integers(0, vocab, size=int(rng.integers(2, 6)))))
        gens[r] = next_gen[0]
        next_gen[0] += 1
        rt.prefill(r, gens[r], prompt, [2 * r, 2 * r + 1])
        tokens[r] = prompt[-1]
        positions[r] = len(prompt) - 1

    for r in range(B):
        start_row(r)

    executed_total = 0
    walls = []
    host_ms = []

    def run_epoch(timed: bool, K: int = K, sink: dict | None = None) -> None:
        nonlocal executed_total
        for r in range(B):
            if positions[r] + K > capacity:
                start_row(r)
        h0 = time.perf_counter()
        out = rt.execute(B, K, tokens, positions, [p + 1 for p in positions], [EOS] * B, gens)
        h1 = time.perf_counter()
        if out.status != 0 or out.device_status != 0:
            raise RuntimeError(f"epoch failed: status={out.status} device={out.device_status}")
        for r in range(B):
            n = int(out.executed[r])
            if n:
                tokens[r] = int(out.token_ids[r, n - 1])
                positions[r] += n
            if n < K:  # EOS: restart the row next epoch
                positions[r] = capacity
        if timed:
            executed_total += int(out.executed.sum())
            walls.append(out.wall_us)
            host_ms.append((h1 - h0) * 1e3)
        if sink is not None:
            sink["executed"] += int(out.executed.sum())
            sink["host_ms"].append((h1 - h0) * 1e3)

    def k_sweep_line(Kx: int, epochs: int) -> dict:
        """tok/s, ms per epoch and per decoder step, and the host-control
        wall of ``epochs`` K=Kx epochs on the same engine and rows (rows that
        would reach the capacity restart before the timed region)."""
        for r in range(B):
            if positions[r] + Kx * (epochs + 2) > capacity:
                start_row(r)
        for _ in range(2):
            run_epoch(False, Kx)
        sink = {"executed": 0, "host_ms": []}
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(epochs):
            run_epoch(False, Kx, sink)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        steps = sink["executed"] / B
        return {"tok_s": round(sink["executed"] / dt, 1), "ms_per_epoch": round(dt * 1e3 / epochs, 4),
                "ms_per_decoder_step": round(dt * 1e3 / steps, 4) if steps else None,
                "host_control_wall_ms_p50": round(statistics.median(sink["host_ms"]), 4), "epochs": epochs,
                "tokens": sink["executed"]}

    import torch

    for _ in range(args.warmup):
        run_epoch(False)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(args.steps):
        run_epoch(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t_start
    # the nodes of one timed epoch's captured graph, counted from the graph
    nodes = {k: rt.info(f"epoch_{k}_nodes") for k in ("memcpy", "memset", "kernel")}
    tok_s = executed_total / elapsed
    ms_per_epoch = elapsed * 1e3 / args.steps
    streamed = rt.info("streamed_weight_bytes")
    decoder_steps = executed_total / B
    ms_per_decoder_step = elapsed * 1e3 / decoder_steps
    step_gbs = streamed / (ms_per_decoder_step * 1e-3) / 1e9
    # every bf16 parameter of the model once per step: the streamed bytes
    # plus the embedding table, of which a step gathers only B rows (Qwen2.5-7B:
    # 15.23 GB against 14.14 GB streamed)
    param_bytes = streamed + rt.vocab * rt.info("hidden") * rt.info("dtype_bytes")
    param_gbs = param_bytes / (ms_per_decoder_step * 1e-3) / 1e9
    # gate/up launched for layer 0, 1, ..., 27 in turn between two HIP events
    # on the engine's stream: every launch streams another layer's 272 MB of
    # weights, so none is warm in the 256 MB memory-side cache, as in the
    # epoch graph (untimed work after the timed epochs)
    k_avg_ms = rt.time_layer_op("gate_up", passes=args.kernel_passes)
    # the same launch inside an epoch, between events around the middle
    # layer's gate/up of each epoch's last step (includes the event overhead)
    rt.enable_kernel_timing(True)
    for _ in range(args.kernel_epochs):
        run_epoch(False)
    torch.cuda.synchronize()
    in_epoch = rt.timed_launch_ms()
    rt.enable_kernel_timing(False)
    # the K sweep (untimed for the headline): the same rows at K = 1, 2, 4
    k_sweep = {}
    if args.sweep_epochs > 0:
        for Kx in (1, 2, 4):
            k_sweep[str(Kx)] = k_sweep_line(Kx, args.sweep_epochs)
            log(f"K={Kx}: {k_sweep[str(Kx)]['tok_s']} tok/s, {k_sweep[str(Kx)]['ms_per_epoch']} ms/epoch, "
                f"host-control wall {k_sweep[str(Kx)]['host_control_wall_ms_p50']} ms")
        k_sweep[str(K)] = {"tok_s": round(tok_s, 1), "ms_per_epoch": round(ms_per_epoch, 4),
                           "ms_per_decoder_step": round(ms_per_decoder_step, 4),
                           "host_control_wall_ms_p50": round(statistics.median(host_ms), 4), "epochs": args.steps,
                           "tokens": executed_total}
    inter = rt.info("intermediate")
    hidden = rt.info("hidden")
    k_bytes = 2 * inter * hidden * 2 + hidden * 2 + B * hidden * 2 + B * inter * 2
    k_name = "gate/up projection (k_proj<bf16,4,4,GateUp>), 28 layers back to back (cold weights)"
    k_gbs = k_bytes / (k_avg_ms * 1e-3) / 1e9
    log(
        f"{tok_s:.1f} tok/s, {ms_per_decoder_step:.3f} ms/decoder step, {step_gbs:.0f} GB/s step, "
        f"gate/up {k_avg_ms * 1e3:.1f} us ({k_gbs:.0f} GB/s)"
    )

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(rt, args.cpu_epochs)
    rt.close()

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_epoch, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 weights generated on the device; random 2-5 token prompts)",
        "config": {
            "workload": "Qwen2.5-7B-shape resident decode epoch, B=4, K=8, block 128 x 2 per row",
            "batch": B,
            "epoch_steps": K,
            "logical_capacity": capacity,
            "bench_step": "one K=8 epoch (8 decoder steps, 4 rows)",
            **({"tuning": json.loads(args.tuning)} if args.tuning else {}),
        },
        "ms_per_decoder_step": round(ms_per_decoder_step, 4),
        "step_weight_stream_gbs": round(step_gbs, 1),
        "step_roofline_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "step_streamed_bytes": streamed,
        "param_bytes": param_bytes,
        "step_param_roofline_frac": round(param_gbs / HBM_PEAK_GBS, 4),
        "host_control_wall_ms_p50": round(statistics.median(host_ms), 4),
        "native_wall_us_p50": int(statistics.median(walls)),
        "epoch_graph_nodes": nodes,
        "k_sweep": k_sweep or None,
        "copy_dispatches_between_epochs_in_trace": epoch_trace_copies(),
        "roofline": {
            "bound": "hbm",
            "kernel": k_name,
            "achieved": round(k_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes(),
            "avg_launch_us": round(k_avg_ms * 1e3, 2),
            "in_epoch_launch_us_with_event_overhead": round(statistics.mean(in_epoch) * 1e3, 2) if in_epoch else None,
            "algorithmic_bytes_per_launch": k_bytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


SCALED_METRIC = "one Qwen2.5-7B layer + LM head, B=64 K=8 epoch decode tok/s; % of HBM roofline (weights + KV)"


def bench_scaled(args) -> int:
    """The scaled-batch workload: one Qwen2.5-7B layer (bf16) and the LM head at
    64 rows, a 1024-block pool of 128-token blocks, 8 random blocks per row,
    contexts uniform in [256, 1016), one K=8 epoch per bench step through the
    8-input/2-output epoch ABI.  Every timed epoch starts from the same
    resident state (rewritten between epochs, outside the timed call), so
    each does the same work."""
    import torch

    from cruise_amd.runtime import (EngineConfig, EngineSpec, ModelSpec, ResidentEpochRuntime, WeightSpec, pack_feed,
                                    tiling_bytes)

    B, P, BS, BPR, CAP, K = 64, 1024, 128, 8, 1024, 8
    cfg = EngineConfig(
        model=ModelSpec(num_layers=1),
        engine=EngineSpec(batch=B, physical_blocks=P, block_size=BS, blocks_per_row=BPR, logical_capacity=CAP),
        weights=WeightSpec(source="synthetic", seed=args.seed, std=0.02),
    )
    t0 = time.time()
    rt = ResidentEpochRuntime(cfg)
    log(f"engine up in {time.time() - t0:.1f}s")
    rng = np.random.default_rng(args.seed + 64)
    table = rng.permutation(P)[: B * BPR].astype(np.int32).reshape(B, BPR)
    pos = rng.integers(256, CAP - K, size=B).astype(np.int64)
    tok = rng.integers(0, rt.vocab, size=B).astype(np.int64)
    gens = np.arange(1, B + 1, dtype=np.int32)
    g = torch.Generator(device="cuda").manual_seed(args.seed)
    kv = (torch.randn(rt.cache_bytes // 2, generator=g, device="cuda") * 0.125).to(torch.bfloat16)
    rt.write_state("key_cache", kv)
    rt.write_state("value_cache", kv)
    del kv
    rows = np.stack([gens, tok, pos, pos + 1, np.ones(B)]).astype(np.int64)
    control = np.zeros(3 + 2 * B, dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = EOS
    control[3 + B :] = gens
    slots = (table[np.arange(B), pos // BS] * BS + pos % BS).astype(np.int32)
    feed = pack_feed(tok, pos, (pos + 1).astype(np.int32), slots, np.ones(B, dtype=np.int32), table, tiling_bytes(),
                     control)
    times, produced = [], 0
    for e in range(args.warmup + args.steps):
        rt.write_state("resident_rows", rows)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        _, ctrl = rt.proc(feed)
        dt = time.perf_counter() - t1
        if ctrl[3] != 0:
            raise RuntimeError(f"epoch failed: device status {ctrl[3]}")
        if e >= args.warmup:
            times.append(dt)
            produced += int(ctrl[6 + 2 * B : 6 + 3 * B].sum())
    elapsed = sum(times)
    tok_s = produced / elapsed
    ms_epoch = 1e3 * elapsed / args.steps
    steps = produced / B
    ms_step = 1e3 * elapsed / steps
    # bytes one decoder step must move: the streamed weights, every row's
    # keys and values over its context (mean context over the epoch), the
    # fp32 logits
    kv_dim = rt.info("kv_heads") * rt.info("head_dim")
    mean_ctx = float(np.mean(pos)) + (K + 1) / 2
    kv_bytes = int(B * mean_ctx * kv_dim * 2 * 2)
    step_bytes = rt.info("streamed_weight_bytes") + kv_bytes + B * rt.vocab * 4
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9
    # the LM head op (its RMSNorm and the matrix-core projection with its
    # per-CU argmax partials), launched alone between HIP events on the
    # engine stream
    if not rt.info("mfma"):
        raise RuntimeError("the 64-row workload expects the matrix-core plan")
    lm_kernel = "k_mf_norm + k_mf_lm_cu (per-CU argmax partials)"
    lm_op = rt.info("step_ops") - 1
    lm_ms = rt.time_ops(lm_op, lm_op + 1, iters=20)
    hidden = rt.info("hidden")
    lm_bytes = rt.vocab * hidden * 2 + B * hidden * 2 * 2 + B * rt.vocab * 4
    lm_gbs = lm_bytes / (lm_ms * 1e-3) / 1e9
    log(f"{tok_s:.0f} tok/s, {ms_step:.3f} ms/decoder step ({step_gbs:.0f} GB/s), LM head {lm_ms * 1e3:.1f} us "
        f"({lm_gbs:.0f} GB/s)")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_scaled(rt, table, tok, pos, gens)
    rt.close()
    print(json.dumps({
        "metric": SCALED_METRIC,
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_epoch, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) bf16 weights and N(0,0.125) KV on the device, random block tables)",
        "config": {"workload": "one Qwen2.5-7B layer + LM head, B=64, K=8, contexts 256-1016, block 128 x 8 per row, "
                               "pool 1024", "batch": B, "epoch_steps": K, "logical_capacity": CAP,
                   "bench_step": "one K=8 epoch (8 decoder steps, 64 rows)"},
        "ms_per_decoder_step": round(ms_step, 4),
        "step_bytes": step_bytes,
        "step_gbs": round(step_gbs, 1),
        "step_roofline_frac": round(step_gbs / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "kernel": f"LM head op ({lm_kernel}), alone",
                     "achieved": round(lm_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(lm_gbs / HBM_PEAK_GBS, 4), "traffic": None, "avg_launch_us": round(lm_ms * 1e3, 2),
                     "algorithmic_bytes_per_launch": lm_bytes},
        "cpu_baseline": cpu,
    }), flush=True)
    return 0


def cpu_baseline_scaled(rt, table, tok, pos, gens):
    """One K=8 epoch of the oracle's controller and PyTorch decoder at the
    scaled batch (one layer, B=64, bf16) from the same resident state, on the
    host cores (weights and caches copied from the engine)."""
    import torch

    from oracle.controller import ControllerGeometry, EpochController, EpochFeed, control_input_elements
    from oracle.decoder import OracleDecoder, PagedGeometry, QWEN25_7B, weight_shapes
    from cruise_amd.runtime import tiling_bytes
    import dataclasses

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    dims = dataclasses.replace(QWEN25_7B, num_layers=1)
    B, P, BS, BPR, CAP, K = 64, 1024, 128, 8, 1024, 8
    weights = {}
    for name, shape in weight_shapes(dims).items():
        t = torch.empty(shape, dtype=torch.bfloat16)
        rt.read_state(name, t)
        weights[name] = t
    geo = PagedGeometry(batch=B, physical_blocks=P, block_size=BS, blocks_per_row=BPR, window=CAP)
    dec = OracleDecoder(dims, geo, weights)
    cg = ControllerGeometry(batch=B, capacity=CAP, physical_blocks=P, blocks_per_row=BPR, block_size=BS,
                            vocab=dims.vocab, num_layers=1)
    ctl = EpochController(cg, dec.forward, dec.cache_shape(), torch.bfloat16)
    k = torch.empty(rt.cache_bytes // 2, dtype=torch.bfloat16)
    v = torch.empty_like(k)
    rt.read_state("key_cache", k)
    rt.read_state("value_cache", v)
    ctl.resident_key, ctl.resident_value = k.view(dec.cache_shape()), v.view(dec.cache_shape())
    ctl.resident_generation = [int(x) for x in gens]
    ctl.resident_token = [int(x) for x in tok]
    ctl.resident_position = [int(x) for x in pos]
    ctl.resident_length = [int(x) + 1 for x in pos]
    ctl.resident_valid = [1] * B
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = EOS
    control[3 + B :] = gens
    slots = (table[np.arange(B), pos // BS] * BS + pos % BS).astype(np.int32)
    feed = EpochFeed(tok.copy(), pos.copy(), (pos + 1).astype(np.int32), slots, np.ones(B, dtype=np.int32),
                     table.reshape(-1), tiling_bytes(), control)
    t1 = time.perf_counter()
    fetch = ctl.proc(feed)
    dt = time.perf_counter() - t1
    produced = int(fetch.control[6 + 2 * B : 6 + 3 * B].sum())
    log(f"cpu baseline (scaled): one K=8 epoch in {dt:.2f}s for {produced} tokens")
    return {"value": round(produced / dt, 2), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"one K=8 epoch of the oracle's controller + PyTorch decoder (one 7B layer + LM head, bf16, "
                      f"B=64, contexts 256-1016) on {cores} threads; {dt:.2f}s for {produced} tokens",
            "epoch_s": round(dt, 3)}


def epoch_trace_copies():
    """Copy dispatches between consecutive epochs (the fetch of one, the feed
    of the next) in the committed kernel-trace summary of this bench, or
    None without it."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "qwen7b_b4_k8_epoch_kernels.json")
    try:
        with open(path) as f:
            return json.load(f)["copy_dispatches_between_epochs"]
    except (OSError, KeyError, ValueError):
        return None


def traffic_bytes():
    """HBM bytes per launch of the reported kernel (gate/up) from the
    committed rocprofv3 PMC passes over the decoder step's kernels
    (FETCH_SIZE and WRITE_SIZE, each scaled by what the counter reads for a
    plain copy of known size; cruise_amd/pmcsummary.py), or None without
    them."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_kernels_qwen7b_b4_traffic.json")
    try:
        with open(path) as f:
            rows = json.load(f)["kernels"]
        return int(next(r["traffic_bytes"] for r in rows if r["op"] == "gate_up"))
    except (OSError, KeyError, ValueError, StopIteration):
        return None


def _cpu_epochs(ctl, tokens, positions, gens, table, K: int, eos: int, warmup: int, epochs: int):
    """``warmup`` then ``epochs`` timed K-step epochs of the oracle controller
    on rows that continue from ``tokens``/``positions`` (updated in place).
    Returns the epoch times and the tokens each produced."""
    from oracle.controller import EpochFeed, control_input_elements
    from cruise_amd.runtime import tiling_bytes

    B, bpr = table.shape
    bs = ctl.geometry.block_size
    control = np.zeros(control_input_elements(B), dtype=np.int32)
    control[0] = K
    control[1 : 1 + B] = eos
    control[3 + B :] = gens
    times, produced = [], []
    for e in range(warmup + epochs):
        slots = np.array([table[r, positions[r] // bs] * bs + positions[r] % bs for r in range(B)], dtype=np.int32)
        feed = EpochFeed(tokens.copy(), positions.copy(), (positions + 1).astype(np.int32), slots,
                         np.ones(B, dtype=np.int32), table.reshape(-1), tiling_bytes(), control)
        t1 = time.perf_counter()
        fetch = ctl.proc(feed)
        dt = time.perf_counter() - t1
        executed = fetch.control[6 + 2 * B : 6 + 3 * B]
        if fetch.control[3] != 0 or (executed == 0).all():
            raise RuntimeError(f"cpu baseline epoch failed: status {fetch.control[3]}")
        for r in range(B):
            if executed[r]:
                tokens[r] = fetch.history[executed[r] - 1, r]
                positions[r] += executed[r]
        if e >= warmup:
            times.append(dt)
            produced.append(int(executed.sum()))
    return times, produced


def _cpu_line(times, produced, K: int) -> dict:
    med = statistics.median(times)
    tok = statistics.median(produced)
    return {"tok_s": round(tok / med, 3), "median_epoch_s": round(med, 4), "ms_per_decoder_step": round(1e3 * med / K, 2),
            "epochs": len(times), "tokens_per_epoch": tok}


def _prefilled_controller(dims, weights, geo_args, B: int, seed: int, prompt_vocab: int):
    """The oracle controller with every row prefilled from a 2-5 token prompt."""
    import torch

    from oracle.controller import ControllerGeometry, EpochController
    from oracle.decoder import OracleDecoder, PagedGeometry

    P, BS, BPR, cap = geo_args
    geo = PagedGeometry(batch=B, physical_blocks=P, block_size=BS, blocks_per_row=BPR, window=cap)
    dec = OracleDecoder(dims, geo, weights)
    cg = ControllerGeometry(batch=B, capacity=cap, physical_blocks=P, blocks_per_row=BPR, block_size=BS,
                            vocab=dims.vocab, num_layers=dims.num_layers)
    ctl = EpochController(cg, dec.forward, dec.cache_shape(), dims.torch_dtype)
    rng = np.random.default_rng(seed)
    table = np.arange(B * BPR, dtype=np.int32).reshape(B, BPR)
    tokens = np.zeros(B, dtype=np.int64)
    positions = np.zeros(B, dtype=np.int64)
    for r in range(B):
        prompt = list(map(int, rng.integers(0, prompt_vocab, size=int(rng.integers(2, 6)))))
        ctl.prefill_row(r, r + 1, prompt, table[r])
        tokens[r], positions[r] = prompt[-1], len(prompt) - 1
    return ctl, table, tokens, positions, np.arange(1, B + 1)


def cpu_baseline(rt, epochs: int, warmup: int = 2):
    """The oracle's CPU decoder path (oracle/controller.py over
    oracle/decoder.py: the reference's controller loop and PyTorch decoder,
    bf16, full 7B shape) on the host cores, run as the bench runs: four rows
    prefilled with 2-5 token prompts, then K=8 epochs of the controller, each
    8 decoder steps for 4 rows; ``warmup`` epochs, then the median of
    ``epochs`` timed epochs.  Weights are copied from the engine.  The same
    rows then continue at K=1, 2 and 4, and the tiny fp32 model (2 layers,
    hidden 256) runs K=2 epochs: the legs of the K sweep."""
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle.decoder import QWEN25_7B, weight_shapes
    from oracle.weights import generate_weights
    from oracle.workloads import C1

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t0 = time.time()
    weights = {}
    for name, shape in weight_shapes(QWEN25_7B).items():
        t = torch.empty(shape, dtype=torch.bfloat16)
        rt.read_state(name, t)
        weights[name] = t
    log(f"cpu baseline: weights on host in {time.time() - t0:.1f}s, {cores} threads")
    B, K = 4, 8
    ctl, table, tokens, positions, gens = _prefilled_controller(QWEN25_7B, weights, (8, 128, 2, 256), B, 7,
                                                                QWEN25_7B.vocab)
    sweep = {}
    times, produced = _cpu_epochs(ctl, tokens, positions, gens, table, K, EOS, warmup, epochs)
    sweep[str(K)] = _cpu_line(times, produced, K)
    med = statistics.median(times)
    tok_per_epoch = statistics.median(produced)
    log(f"cpu baseline: {epochs} timed K=8 epochs, median {med:.3f}s for {tok_per_epoch} tokens")
    for Kx in (1, 2, 4):
        sweep[str(Kx)] = _cpu_line(*_cpu_epochs(ctl, tokens, positions, gens, table, Kx, EOS, warmup, epochs), Kx)
        log(f"cpu baseline: K={Kx}: {sweep[str(Kx)]['tok_s']} tok/s")
    del ctl, weights
    tiny_w = generate_weights(C1.dims, C1.seed)
    g = C1.geometry
    tctl, ttable, ttok, tpos, tgens = _prefilled_controller(C1.dims, tiny_w, (g.physical_blocks, g.block_size,
                                                            g.blocks_per_row, g.window), g.batch, C1.seed, C1.dims.vocab)
    tiny = _cpu_line(*_cpu_epochs(tctl, ttok, tpos, tgens, ttable, 2, C1.eos, warmup, epochs), 2)
    log(f"cpu baseline: tiny fp32 K=2: {tiny['tok_s']} tok/s")
    cpu_name = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(tok_per_epoch / med, 3),
        "unit": "tok/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"the oracle's controller + PyTorch decoder (bf16, full 7B shape, B=4) on {cores} threads of "
                   f"{cpu_name}: {warmup} warm-up then {epochs} timed K=8 epochs after 2-5 token prompts; "
                   f"median epoch {med:.3f}s for {tok_per_epoch} tokens"),
        "median_epoch_s": round(med, 4),
        "k_sweep": sweep,
        "tiny_fp32_k2": dict(tiny, model="2 layers, hidden 256, GQA 4/2, head_dim 64, vocab 4096, fp32, B=4"),
    }


if __name__ == "__main__":
    sys.exit(main())
