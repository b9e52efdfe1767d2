"""Throughput of the batched prefill (resident_epoch_prefill_batch) on the
Qwen2.5-7B shape with synthetic weights generated on the device.

    python -m cruise_amd.prefillbench --rows 64 --len 1000 --window 1024
    python -m cruise_amd.prefillbench --rows 4 --len 256 --window 256

Every row gets a random prompt of --len tokens; positions 0..len-2 are
prefilled (the last token starts the first epoch), so one call computes
rows x (len - 1) tokens through every layer.  Reported per call: wall time,
tokens/s, and the algorithmic FLOP rate against MI355X's dense bf16 MFMA
peak (2.5 PFLOP/s): 2 x 233,046,016 linear parameters per token per layer
plus the causal attention's 4 x (position + 1) x head_dim x heads per token
per layer (Q K^T and P V).
"""
from __future__ import annotations

import argparse
import json
import time

import numpy as np

LINEAR_PARAMS_PER_LAYER = 233_046_016  # q/k/v, o, gate, up, down of Qwen2.5-7B
MFMA_BF16_PEAK = 2.5e15


def prefill_flops(rows: int, length: int, layers: int, heads: int = 28, head_dim: int = 128) -> float:
    tokens = rows * (length - 1)
    attn = sum(4 * (p + 1) * head_dim * heads for p in range(length - 1)) * rows
    return float(layers) * (2.0 * LINEAR_PARAMS_PER_LAYER * tokens + attn)


def main(argv=None) -> None:
    p = argparse.ArgumentParser()
    p.add_argument("--rows", type=int, default=64)
    p.add_argument("--len", type=int, default=1000, help="prompt tokens per row")
    p.add_argument("--layers", type=int, default=28)
    p.add_argument("--window", type=int, default=1024, help="logical capacity (a multiple of 128)")
    p.add_argument("--iters", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--seed", type=int, default=7)
    p.add_argument("--tuning", default="{}", help='launch-plan overrides as JSON, e.g. {"attention_split": 1}')
    args = p.parse_args(argv)
    if args.window % 128 or not 2 <= args.len <= args.window:
        raise SystemExit("--window must be a multiple of 128 and 2 <= --len <= --window")

    import torch  # noqa: F401  (the library binds torch's HIP runtime)

    from cruise_amd.runtime import EngineConfig, EngineSpec, ModelSpec, ResidentEpochRuntime, WeightSpec

    bpr = args.window // 128
    cfg = EngineConfig(
        model=ModelSpec(num_layers=args.layers),
        engine=EngineSpec(batch=args.rows, physical_blocks=args.rows * bpr, block_size=128, blocks_per_row=bpr,
                          logical_capacity=args.window),
        weights=WeightSpec("synthetic", args.seed, 0.02),
        tuning=json.loads(args.tuning),
    )
    t0 = time.perf_counter()
    rt = ResidentEpochRuntime(cfg)
    print(f"[prefill] engine up in {time.perf_counter() - t0:.1f}s", flush=True)
    try:
        rng = np.random.default_rng(args.seed)
        vocab = rt.vocab
        prompts = [list(map(int, rng.integers(0, vocab, size=args.len))) for _ in range(args.rows)]
        table = np.arange(args.rows * bpr, dtype=np.int32).reshape(args.rows, bpr)
        rows = list(range(args.rows))
        times = []
        for i in range(args.warmup + args.iters):
            t0 = time.perf_counter()
            rt.prefill_batch(rows, [1 + i * args.rows + r for r in rows], prompts, table)
            dt = time.perf_counter() - t0
            if i >= args.warmup:
                times.append(dt)
            print(f"[prefill] call {i}: {dt * 1e3:.1f} ms", flush=True)
        best = min(times)
        tokens = args.rows * (args.len - 1)
        flops = prefill_flops(args.rows, args.len, args.layers)
        print(json.dumps({
            "workload": f"Qwen2.5-7B-shape batched prefill, {args.rows} rows x {args.len} tokens, {args.layers} layers",
            "tokens_per_call": tokens,
            "ms_per_call_min": round(best * 1e3, 2),
            "ms_per_call_median": round(float(np.median(times)) * 1e3, 2),
            "tokens_per_s": round(tokens / best, 1),
            "tflops": round(flops / best / 1e12, 1),
            "mfma_bf16_peak_frac": round(flops / best / MFMA_BF16_PEAK, 4),
        }), flush=True)
    finally:
        rt.close()


if __name__ == "__main__":
    main()
