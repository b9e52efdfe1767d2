"""Time single launches of the decoder step on the Qwen2.5-7B shape.

``python -m cruise_amd.opbench`` builds an engine with synthetic N(0, 0.02)
bf16 weights (generated on the device), runs one decoder step with every row
at ``--context`` tokens (KV cache filled with random values) and then times
the requested launches of the step's launch list eagerly with HIP events
(``resident_epoch_time_ops``): mean microseconds per launch and the
algorithmic HBM bytes each launch must move (weights + activations), i.e.
its achieved bandwidth.

``--copy-bytes N`` instead times a plain device-to-device copy of N bytes
(torch), the calibration kernel for HBM traffic counters.

Examples::

    python -m cruise_amd.opbench                       # every op of layer 3 + LM head
    python -m cruise_amd.opbench --op gate_up --iters 5
    python -m cruise_amd.opbench --copy-bytes 1073741824
    python -m cruise_amd.opbench --op attention --batch 64 --capacity 4096 --context 4096

``--batch`` and ``--capacity`` set the rows and the window (blocks of 128);
``--tuning`` takes the engine's launch-plan overrides, e.g.
``'{"attention_split": 0}'``.
"""
from __future__ import annotations

import argparse
import json
import sys

import numpy as np

OPS = ("qkv", "attention", "o_proj", "o_reduce", "gate_up", "down", "down_reduce")


def algorithmic_bytes(op: str, B: int, H: int, I: int, V: int, qkv_rows: int, kv_dim: int, ctx: int, T: int = 2) -> int:
    """HBM bytes one launch must move at least: weights once, activations in
    and out once (KV: the context's keys and values of one layer)."""
    if op == "qkv":
        return qkv_rows * H * T + qkv_rows * T + B * H * T + B * qkv_rows * T
    if op == "attention":
        return 2 * B * ctx * kv_dim * T + 2 * B * H * T
    if op == "o_proj":
        return H * H * T + B * H * T + B * H * 4
    if op in ("o_reduce", "down_reduce"):
        segments = 1 if op == "o_reduce" else -(-I // 3584)
        return segments * B * H * 4 + 3 * B * H * T + H * T
    if op == "gate_up":
        return 2 * I * H * T + H * T + B * H * T + B * I * T
    if op == "down":
        return H * I * T + B * I * T + -(-I // 3584) * B * H * 4
    if op == "lm_head":
        return V * H * T + B * H * T + B * V * 4
    raise KeyError(op)


def copy_calibration(nbytes: int, iters: int) -> None:
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.random_(0, 255)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        dst.copy_(src)
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / iters
    print(f"copy {nbytes} bytes: {ms * 1e3:.1f} us, {2 * nbytes / (ms * 1e-3) / 1e9:.0f} GB/s (read + write)", flush=True)


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--op", action="append", choices=OPS + ("lm_head", "layer", "step"), help="launch(es) to time (default: all)")
    p.add_argument("--layer", type=int, default=3)
    p.add_argument("--iters", type=int, default=20)
    p.add_argument("--context", type=int, default=128, help="tokens per row already in the KV cache")
    p.add_argument("--copy-bytes", type=int, default=0)
    p.add_argument("--tuning", default="", help="JSON object of launch-plan overrides")
    p.add_argument("--capacity", type=int, default=256, help="window positions per row (a multiple of 128)")
    p.add_argument("--batch", type=int, default=4, help="rows")
    args = p.parse_args()
    if args.copy_bytes:
        copy_calibration(args.copy_bytes, args.iters)
        return 0

    import torch

    from cruise_amd.runtime import EngineConfig, EngineSpec, ModelSpec, ResidentEpochRuntime, WeightSpec

    capacity = args.capacity
    if capacity < 128 or capacity % 128 != 0:
        raise SystemExit("--capacity must be a positive multiple of 128")
    if not 1 <= args.context <= capacity:
        raise SystemExit(f"--context must be in [1, {capacity}]")
    bpr = capacity // 128
    nb = args.batch
    if nb < 1:
        raise SystemExit("--batch must be positive")
    cfg = EngineConfig(
        model=ModelSpec(),
        engine=EngineSpec(
            batch=nb, physical_blocks=nb * bpr, block_size=128, blocks_per_row=bpr, logical_capacity=capacity
        ),
        weights=WeightSpec("synthetic", 1, 0.02),
        tuning=json.loads(args.tuning) if args.tuning else {},
    )
    rt = ResidentEpochRuntime(cfg)
    try:
        B, V = rt.batch, rt.vocab
        H, I = rt.info("hidden"), rt.info("intermediate")
        heads, kv_heads, d = rt.info("heads"), rt.info("kv_heads"), rt.info("head_dim")
        kv_dim = kv_heads * d
        qkv_rows = heads * d + 2 * kv_dim
        ctx = args.context
        table = np.arange(B * bpr, dtype=np.int32).reshape(B, bpr)
        pos = np.full(B, ctx - 1, np.int64)
        ln = np.full((B, 1), ctx, np.int32)
        slot = np.array([table[r, (ctx - 1) // 128] * 128 + (ctx - 1) % 128 for r in range(B)], dtype=np.int32)
        gen = torch.Generator(device="cuda").manual_seed(5)
        kc = (torch.randn(rt.cache_bytes // 2, generator=gen, device="cuda") * 0.125).to(torch.bfloat16)
        vc = (torch.randn(rt.cache_bytes // 2, generator=gen, device="cuda") * 0.125).to(torch.bfloat16)
        logits = torch.zeros(B, V, device="cuda")
        nxt = torch.zeros(B, dtype=torch.int64, device="cuda")
        tok = np.arange(1, B + 1, dtype=np.int64).reshape(B, 1)
        rt.decoder_step(tok, pos, ln, kc, slot, np.ones(B, np.int32), table, vc, logits, nxt)
        ops = args.op or list(OPS) + ["lm_head"]
        print(f"Qwen2.5-7B shape, B={B}, context {ctx}, layer {args.layer}, {args.iters} eager launches each", flush=True)
        print(f"{'op':12s} {'us/launch':>10s} {'MB/launch':>10s} {'GB/s':>8s}", flush=True)
        for op in ops:
            if op == "layer":
                a, b = rt.op_index(args.layer, "qkv"), rt.op_index(args.layer + 1, "qkv")
                nbytes = sum(algorithmic_bytes(o, B, H, I, V, qkv_rows, kv_dim, ctx) for o in OPS)
            elif op == "step":
                a, b = 0, rt.info("step_ops")
                nbytes = rt.info("streamed_weight_bytes")
            else:
                a = rt.op_index(args.layer, op) if op in OPS else rt.op_index(0, op)
                b = a + 1
                nbytes = algorithmic_bytes(op, B, H, I, V, qkv_rows, kv_dim, ctx)
            ms = rt.time_ops(a, b, args.iters)
            print(f"{op:12s} {ms * 1e3:10.1f} {nbytes / 1e6:10.2f} {nbytes / (ms * 1e-3) / 1e9:8.0f}", flush=True)
    finally:
        rt.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
