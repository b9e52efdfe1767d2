"""Shared helpers of the parity tests: engine construction from a workload,
the oracle twin of an engine, and the comparison rules.

Comparison rules (the bar for this path):
* integer and index state (tokens, history, control record, slots, next
  positions, unaddressed KV) -- bit-exact;
* floating point (logits, written KV) -- max |a - b| <= REL_TOL * max |b|
  with REL_TOL = 2e-2 for bf16, tighter for the fp32 model;
* greedy tokens -- equal wherever the oracle's top-2 margin exceeds
  REL_TOL * max |logit| of that row; elsewhere the oracle is teacher-forced
  with the GPU's token so a near-tie does not cascade.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import torch

from cruise_amd.runtime import EngineConfig, EngineSpec, ModelSpec, ResidentEpochRuntime, WeightSpec
from oracle.controller import ControllerGeometry, EpochController
from oracle.decoder import OracleDecoder
from oracle.workloads import Workload

REL_TOL_BF16 = 2e-2
REL_TOL_FP32 = 2e-3


def rel_tol(dims) -> float:
    return REL_TOL_FP32 if dims.dtype == "fp32" else REL_TOL_BF16


def engine_config(w: Workload, *, capacity: int | None = None, weights: WeightSpec | None = None) -> EngineConfig:
    d, g = w.dims, w.geometry
    return EngineConfig(
        model=ModelSpec(
            num_layers=d.num_layers,
            hidden=d.hidden,
            num_heads=d.num_heads,
            num_kv_heads=d.num_kv_heads,
            head_dim=d.head_dim,
            intermediate=d.intermediate,
            vocab=d.vocab,
            rope_theta=d.rope_theta,
            rms_eps=d.rms_eps,
            dtype=d.dtype,
        ),
        engine=EngineSpec(
            batch=g.batch,
            physical_blocks=g.physical_blocks,
            block_size=g.block_size,
            blocks_per_row=g.blocks_per_row,
            logical_capacity=capacity if capacity is not None else g.window,
            configured_eos=w.eos,
        ),
        weights=weights or WeightSpec("upload"),
    )


def make_runtime(w: Workload, weights: dict, *, capacity: int | None = None, tuning: dict | None = None) -> ResidentEpochRuntime:
    cfg = engine_config(w, capacity=capacity)
    if tuning:
        cfg = replace(cfg, tuning=dict(tuning))
    rt = ResidentEpochRuntime(cfg, weights=weights)
    # RoPE frequencies exactly as the oracle computes them (fp32 torch pow).
    from oracle.decoder import inv_freq

    rt.write_state("inv_freq", inv_freq(w.dims).contiguous())
    return rt


def oracle_controller(w: Workload, weights_cpu: dict, *, capacity: int | None = None) -> tuple[OracleDecoder, EpochController]:
    g = w.geometry
    cap = capacity if capacity is not None else g.window
    from oracle.decoder import PagedGeometry

    geo = PagedGeometry(g.batch, g.physical_blocks, g.block_size, g.blocks_per_row, cap)
    dec = OracleDecoder(w.dims, geo, weights_cpu)
    cg = ControllerGeometry(
        batch=g.batch,
        capacity=cap,
        physical_blocks=g.physical_blocks,
        blocks_per_row=g.blocks_per_row,
        block_size=g.block_size,
        vocab=w.dims.vocab,
        num_layers=w.dims.num_layers,
    )
    ctl = EpochController(cg, dec.forward, dec.cache_shape(), w.dims.torch_dtype)
    return dec, ctl


def engine_snapshot(rt: ResidentEpochRuntime, dtype: torch.dtype) -> tuple:
    """The engine's resident state (caches on the device, resident rows)."""
    elems = rt.cache_bytes // torch.tensor([], dtype=dtype).element_size()
    k = torch.empty(elems, dtype=dtype, device="cuda")
    v = torch.empty(elems, dtype=dtype, device="cuda")
    rt.read_state("key_cache", k)
    rt.read_state("value_cache", v)
    return k, v, rt.resident_rows().copy()


def engine_restore(rt: ResidentEpochRuntime, snap: tuple) -> None:
    k, v, rows = snap
    rt.write_state("key_cache", k)
    rt.write_state("value_cache", v)
    rt.write_state("resident_rows", rows)


def oracle_snapshot(ctl: EpochController) -> dict:
    return {
        "key": ctl.resident_key.clone(),
        "value": ctl.resident_value.clone(),
        "rows": [list(ctl.resident_generation), list(ctl.resident_token), list(ctl.resident_position),
                 list(ctl.resident_length), list(ctl.resident_valid)],
    }


def oracle_restore(ctl: EpochController, snap: dict) -> None:
    ctl.resident_key = snap["key"].clone()
    ctl.resident_value = snap["value"].clone()
    (ctl.resident_generation, ctl.resident_token, ctl.resident_position, ctl.resident_length,
     ctl.resident_valid) = (list(r) for r in snap["rows"])


def first_max(row: np.ndarray) -> int:
    """First index of the maximum (numpy's argmax returns the first occurrence)."""
    return int(np.argmax(np.asarray(row, dtype=np.float32)))


def assert_close_rel(actual, expected, rel: float, what: str) -> None:
    a = torch.as_tensor(actual).float()
    b = torch.as_tensor(expected).float()
    assert a.shape == b.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(b.shape)}"
    assert torch.isfinite(a).all(), f"{what}: non-finite values"
    scale = float(b.abs().max())
    err = float((a - b).abs().max())
    assert err <= rel * max(scale, 1e-30), f"{what}: max|diff|={err:.3e} > {rel} * max|ref|={scale:.3e}"


def top2_margin(row: np.ndarray) -> float:
    part = np.partition(row.astype(np.float64), -2)[-2:]
    return float(part[1] - part[0])


class TeacherForcing:
    """Token override for the oracle controller: checks the GPU token against
    the oracle's argmax where the margin is decisive, then forces the GPU's
    token so both sides continue on the same sequence."""

    def __init__(self, gpu_history: np.ndarray, rel: float):
        self.gpu = gpu_history
        self.rel = rel
        self.checked = 0
        self.forced = 0
        self.mismatches: list = []

    def __call__(self, step: int, row: int, oracle_token: int, logits_row: np.ndarray) -> int:
        gpu_token = int(self.gpu[step, row])
        if gpu_token < 0:  # the GPU did not run this row at this step
            self.mismatches.append((step, row, gpu_token, oracle_token, None))
            return oracle_token
        margin = top2_margin(logits_row)
        decisive = margin > self.rel * float(np.abs(logits_row).max())
        if decisive:
            self.checked += 1
            if gpu_token != oracle_token:
                self.mismatches.append((step, row, gpu_token, oracle_token, margin))
        elif gpu_token != oracle_token:
            self.forced += 1
        return gpu_token
