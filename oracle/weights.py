"""Seeded synthetic weights in the reference bundle naming.

Oracle (test infrastructure only).  Every tensor is drawn N(0, std) in fp32
from one ``torch.Generator`` seeded with ``seed``, in the bundle order of
materialize_runtime_weights.py:53-80 (embedding, then per layer the twelve
tensors, then final norm and LM head), and cast to the model dtype.  The
generator may live on the GPU (``device="cuda"``) for the 7B shapes; the
values are then copied to the host for the oracle, so both sides hold the
same numbers whatever the generator.
"""
from __future__ import annotations

import torch

from .decoder import ModelDims, weight_shapes


def generate_weights(
    dims: ModelDims, seed: int, std: float = 0.02, device: str = "cpu"
) -> dict[str, torch.Tensor]:
    generator = torch.Generator(device=device).manual_seed(seed)
    out: dict[str, torch.Tensor] = {}
    for name, shape in weight_shapes(dims).items():
        draw = torch.randn(shape, generator=generator, dtype=torch.float32, device=device)
        out[name] = (draw * std).to(dims.torch_dtype)
        del draw
    return out


def seeded_cache(shape: tuple[int, ...], seed: int, dtype: torch.dtype, scale: float = 0.125):
    """KV contents ``randn * 0.125`` from a seed, as the reference's B=4 gate
    (history/attempts/g4c-attempt69b-b4-eager/b4_eager_test.py:61-76)."""
    generator = torch.Generator(device="cpu").manual_seed(seed)
    key = (torch.randn(shape, generator=generator, dtype=torch.float32) * scale).to(dtype)
    value = (torch.randn(shape, generator=generator, dtype=torch.float32) * scale).to(dtype)
    return key, value
