"""The batched-prefill GEMM through resident_epoch_gemm, against a plain
matrix product of the same operands on the CPU, at shapes with partial tiles
in M and N (the bf16 kernel's tiles are 256 x 256, 256 x 128 for the SwiGLU
epilogue) and for every epilogue:

* integer-valued operands (|a|, |w| <= 2 and K <= 3584 keep every partial sum
  an integer below 2^24, so fp32 sums are exact in any order): the store and
  residual epilogues must equal the CPU product bit for bit, which pins the
  tile indexing, the operand layout and the rounding points exactly; the
  SwiGLU epilogue within two bf16 steps (its exp is the device's expf, the
  reference's the CPU's);
* random operands: within two bf16 rounding steps of the magnitudes involved
  (the fp32 summation orders differ, and a residual or bias add can round a
  one-step difference of the product again);
* shapes the bf16 kernel does not take are refused with -1.

The model's own shapes are covered by the prefill tests against the oracle."""
from __future__ import annotations

import ctypes

import pytest
import torch

from cruise_amd import _lib

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
SHAPES = [(1, 8, 64), (300, 264, 192), (513, 520, 128), (257, 136, 3584)]


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def run(lib, A, W, W2, bias, out, epilogue):
    M, K = A.shape
    N = W.shape[0]
    dtype_bytes = A.element_size()
    return lib.resident_epoch_gemm(ptr(A), ptr(W), ptr(W2), ptr(bias), ptr(out), M, N, K, epilogue, dtype_bytes)


def reference(A, W, W2, bias, out0, epilogue):
    """fp32 products on the CPU with the kernel's rounding points."""
    T = A.dtype
    r = lambda x: x.to(T).float()
    y = A.float() @ W.float().T
    if epilogue == 0:
        return (y + (bias.float() if bias is not None else 0.0)).to(T)
    if epilogue == 1:
        return (out0.float() + r(y)).to(T)
    g = r(y)
    u = r(A.float() @ W2.float().T)
    return (r(g / (1.0 + torch.exp(-g))) * u).to(T)


def operands(M, N, K, dtype, integer, seed):
    gen = torch.Generator().manual_seed(seed)
    if integer:
        mk = lambda *s: torch.randint(-2, 3, s, generator=gen).to(dtype)
        return mk(M, K), mk(N, K), mk(N, K), mk(N), mk(M, N)
    A = torch.randn(M, K, generator=gen).to(dtype)
    W = (torch.randn(N, K, generator=gen) / K ** 0.5).to(dtype)
    W2 = (torch.randn(N, K, generator=gen) / K ** 0.5).to(dtype)
    return A, W, W2, torch.randn(N, generator=gen).to(dtype), torch.randn(M, N, generator=gen).to(dtype)


def one(lib, M, N, K, dtype, epilogue, integer, seed, with_bias=True):
    A, W, W2, bias, out0 = operands(M, N, K, dtype, integer, seed)
    if not with_bias:
        bias = None
    dev = lambda t: t.cuda() if t is not None else None
    out = dev(out0).clone()
    rc = run(lib, dev(A), dev(W), dev(W2) if epilogue == 2 else None, dev(bias), out, epilogue)
    torch.cuda.synchronize()
    assert rc == 0, rc
    return out.cpu(), reference(A, W, W2, bias, out0, epilogue)


def within_two_steps(got, ref, A, W, W2):
    g, r = got.float(), ref.float()
    mag = torch.maximum(r.abs(), (A.float() @ W.float().T).abs())
    mag = torch.maximum(mag, (A.float() @ W2.float().T).abs())
    tol = torch.clamp(mag, min=1.0) * 2.0 ** -6
    bad = (g - r).abs() > tol
    assert not bad.any(), f"{bad.sum().item()} of {r.numel()} outputs off by more than two bf16 steps"


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("epilogue", [0, 1, 2])
def test_bf16_gemm_integer_operands(lib, M, N, K, epilogue):
    seed = M + N + K + epilogue
    got, ref = one(lib, M, N, K, BF16, epilogue, True, seed)
    if epilogue < 2:
        assert torch.equal(got, ref), f"{(got != ref).sum().item()} of {ref.numel()} outputs differ"
    else:
        A, W, W2, _, _ = operands(M, N, K, BF16, True, seed)
        within_two_steps(got, ref, A, W, W2)


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("epilogue", [0, 1, 2])
def test_bf16_gemm_random_operands(lib, M, N, K, epilogue):
    seed = 7 * (M + N + K) + epilogue
    got, ref = one(lib, M, N, K, BF16, epilogue, False, seed)
    A, W, W2, _, _ = operands(M, N, K, BF16, False, seed)
    within_two_steps(got, ref, A, W, W2)


def test_bf16_gemm_store_without_bias(lib):
    got, ref = one(lib, 300, 264, 192, BF16, 0, True, seed=3, with_bias=False)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("M,N,K", [(1, 8, 16), (300, 264, 192), (70, 65, 33)])
@pytest.mark.parametrize("epilogue", [0, 1])
def test_fp32_gemm_exact_on_integer_operands(lib, M, N, K, epilogue):
    got, ref = one(lib, M, N, K, torch.float32, epilogue, True, seed=M * N + K + epilogue)
    assert torch.equal(got, ref)


def test_bf16_gemm_refuses_shapes_it_does_not_take(lib):
    A = torch.zeros(16, 96, dtype=BF16, device="cuda")
    W = torch.zeros(16, 96, dtype=BF16, device="cuda")
    out = torch.zeros(16, 16, dtype=BF16, device="cuda")
    assert run(lib, A, W, None, None, out, 0) == -1  # K % 64 != 0
    A = torch.zeros(16, 64, dtype=BF16, device="cuda")
    W = torch.zeros(12, 64, dtype=BF16, device="cuda")
    out = torch.zeros(16, 12, dtype=BF16, device="cuda")
    assert run(lib, A, W, None, None, out, 0) == -1  # N % 8 != 0
    W = torch.zeros(16, 64, dtype=BF16, device="cuda")
    out = torch.zeros(16, 16, dtype=BF16, device="cuda")
    assert run(lib, A, W, None, None, out, 2) == -1  # SwiGLU without the up rows
    assert run(lib, A, W, None, None, out, 3) == -1  # no such epilogue
    torch.cuda.synchronize()
