"""kch_linear_rows (decode-step projections) against an fp32 torch reference.

y = x w^T with x [M, K], w [N, K] in bf16 / fp16 and fp32 accumulation; the
result is rounded once to the input dtype, so it must agree with the fp32
product of the same (already rounded) inputs to within that rounding plus the
accumulation-order difference.
"""

from __future__ import annotations

import pytest
import torch

from kch import _lib

pytestmark = pytest.mark.gpu


def _run(x, w, y):
    M, K = x.shape
    N = w.shape[0]
    _lib.call("kch_linear_rows", _lib.ptr(x), x.stride(0), _lib.ptr(w), w.stride(0), _lib.ptr(y),
              y.stride(0), M, N, K, _lib.dtype_code("test", x.dtype), _lib.stream_of(x))
    torch.cuda.synchronize()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (2, 6288, 2048), (5, 100, 128), (16, 2048, 2048),
                                   (3, 33, 4096), (2, 2048, 128)])
def test_linear_rows_matches_fp32(dev, dt, M, N, K):
    g = torch.Generator(device="cpu").manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, generator=g).to(dev, dt)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev, dt)
    y = torch.full((M, N), float("nan"), device=dev, dtype=dt)
    _run(x, w, y)
    ref = x.float() @ w.float().t()
    err = (y.float() - ref).abs()
    tol = 8e-3 * ref.abs() + 2e-3 * ref.abs().max()
    assert bool(torch.isfinite(y.float()).all())
    assert bool((err <= tol).all()), float(err.max())


def test_linear_rows_strided_rows_and_output(dev):
    # x rows inside a wider buffer (a slice of a fused projection), y rows padded
    M, N, K = 3, 70, 256
    g = torch.Generator(device="cpu").manual_seed(3)
    big = torch.randn(M, K + 64, generator=g).to(dev, torch.bfloat16)
    x = big[:, 32:32 + K]
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev, torch.bfloat16)
    yb = torch.full((M, N + 10), 7.0, device=dev, dtype=torch.bfloat16)
    y = yb[:, :N]
    _run(x, w, y)
    ref = x.float() @ w.float().t()
    assert float((y.float() - ref).abs().max()) <= 1e-2 * float(ref.abs().max())
    assert bool((yb[:, N:] == 7.0).all())  # nothing written past N


def test_linear_rows_in_hybrid_decode_matches_f_linear(dev):
    # the hybrid decode helper picks the kernel for <= 16 rows and F.linear otherwise
    from kch import hybrid
    g = torch.Generator(device="cpu").manual_seed(9)
    w = (torch.randn(512, 2048, generator=g) / 45.0).to(dev, torch.bfloat16)
    for rows in (1, 2, 16, 17):
        x = torch.randn(rows, 1, 2048, generator=g).to(dev, torch.bfloat16)
        y = hybrid._linear(x, w)
        ref = torch.nn.functional.linear(x.float(), w.float())
        assert tuple(y.shape) == (rows, 1, 512)
        assert float((y.float() - ref).abs().max()) <= 1e-2 * float(ref.abs().max())


def test_linear_rows_in_hybrid_decode_views(dev):
    # column slices of a wider input and row slices of a wider weight take the
    # strided path; a one-row weight view takes the contiguous one
    from kch import hybrid
    g = torch.Generator(device="cpu").manual_seed(10)
    xw = torch.randn(3, 1, 2048 + 256, generator=g).to(dev, torch.bfloat16)
    ww = (torch.randn(700, 2048, generator=g) / 45.0).to(dev, torch.bfloat16)
    cases = [(xw[..., :2048], ww[:512]), (xw[..., 64:64 + 2048], ww[8:520]),
             (xw[..., :2048].contiguous(), ww[5:6]), (xw[..., 256:], ww[:, :2048])]
    for x, w in cases:
        y = hybrid._linear(x, w)
        ref = torch.nn.functional.linear(x.float(), w.float())
        assert tuple(y.shape) == (3, 1, w.shape[0])
        assert float((y.float() - ref).abs().max()) <= 1e-2 * float(ref.abs().max())


def _run_up(x, w, y):
    M, K = x.shape
    N = w.shape[0]
    _lib.call("kch_linear_up", _lib.ptr(x), x.stride(0), _lib.ptr(w), w.stride(0), _lib.ptr(y),
              y.stride(0), M, N, K, _lib.dtype_code("test", x.dtype), _lib.stream_of(x))
    torch.cuda.synchronize()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N,K", [(1, 16, 32), (63, 2048, 128), (64, 2304, 128), (1000, 100, 64),
                                   (4097, 2048, 256), (131072, 2048, 128), (77, 8, 32)])
def test_linear_up_matches_fp32(dev, dt, M, N, K):
    """kch_linear_up (the prefill query up-projection) against the fp32 product
    of the same inputs, every element."""
    g = torch.Generator(device="cpu").manual_seed(M + 3 * N + K)
    x = torch.randn(M, K, generator=g).to(dev, dt)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev, dt)
    y = torch.full((M, N), float("nan"), device=dev, dtype=dt)
    _run_up(x, w, y)
    ref = x.float() @ w.float().t()
    err = (y.float() - ref).abs()
    tol = 8e-3 * ref.abs() + 2e-3 * ref.abs().max()
    assert bool(torch.isfinite(y.float()).all())
    assert bool((err <= tol).all()), float(err.max())


def test_linear_up_strided(dev):
    # x: the latent columns of a fused projection output; y rows padded
    M, N, K = 300, 2304, 128
    g = torch.Generator(device="cpu").manual_seed(5)
    big = torch.randn(M, 384 + K, generator=g).to(dev, torch.bfloat16)
    x = big[:, 384:384 + K]
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dev, torch.bfloat16)
    yb = torch.full((M, N + 16), 7.0, device=dev, dtype=torch.bfloat16)
    y = yb[:, :N]
    _run_up(x, w, y)
    ref = x.float() @ w.float().t()
    assert float((y.float() - ref).abs().max()) <= 1e-2 * float(ref.abs().max())
    assert bool((yb[:, N:] == 7.0).all())

