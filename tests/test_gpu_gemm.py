"""hsl_gemm_f32 (fp32 MFMA GEMM) against an fp64 CPU product.

Tolerance: the fp32 result must lie within 2e-6 * sqrt(K) * (|A| |B|)_mn of the
fp64 product (|A||B| is the product of absolute values, the scale of the
rounding error of any fp32 summation order).
"""

import pytest
import torch

from prlstm_amd import _lib

pytestmark = pytest.mark.gpu


def _gemm(A, B, bias, M, N, K, ta, tb, split=True):
    dev = A.device
    C = torch.empty(M, N, device=dev)
    lda, ldb = max(A.shape[1], 1), max(B.shape[1], 1)
    nbytes = _lib.load().hsl_gemm_ws_bytes(M, N, K) if split else 0
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    P = _lib.ptr
    _lib.call("hsl_gemm_f32", P(A), P(B), P(bias), P(C), M, N, K, lda, ldb, N, int(ta), int(tb),
              P(ws), nbytes, _lib.stream_of(dev))
    return C


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 7, 3), (33, 65, 17), (128, 128, 32),
                                   (96, 48, 8192), (300, 200, 130), (2048, 512, 4096)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_matches_fp64(dev, M, N, K, ta, tb):
    print(f"gemm M={M} N={N} K={K} ta={ta} tb={tb}", flush=True)
    g = torch.Generator().manual_seed(M * 31 + N * 7 + K + ta * 2 + tb)
    a = torch.randn(M, K, generator=g)
    b = torch.randn(K, N, generator=g)
    bias = torch.randn(N, generator=g)
    A = (a.t().contiguous() if ta else a).to(dev)
    B = (b.t().contiguous() if tb else b).to(dev)
    C = _gemm(A, B, bias.to(dev), M, N, K, ta, tb).cpu().double()
    ref = a.double() @ b.double() + bias.double()
    scale = a.double().abs() @ b.double().abs() + bias.double().abs()
    err = (C - ref).abs()
    assert bool((err <= 2e-6 * max(K, 1) ** 0.5 * scale + 1e-30).all()), float((err / scale).max())


def test_gemm_split_and_unsplit_agree(dev):
    M, N, K = 256, 256, 16384
    g = torch.Generator().manual_seed(0)
    a = torch.randn(K, M, generator=g).to(dev)
    b = torch.randn(K, N, generator=g).to(dev)
    c1 = _gemm(a, b, None, M, N, K, 1, 0, split=True)
    c2 = _gemm(a, b, None, M, N, K, 1, 0, split=False)
    ref = a.cpu().double().t() @ b.cpu().double()
    e1 = (c1.cpu().double() - ref).abs().max().item()
    e2 = (c2.cpu().double() - ref).abs().max().item()
    print(f"split err {e1:.3e} unsplit err {e2:.3e}")
    assert e1 < 5e-3 and e2 < 5e-3


def test_gemm_empty_and_unaligned(dev):
    # K = 0 gives the bias; an offset (non 16-byte aligned) view takes the scalar path
    z = torch.zeros(3, 0, device=dev)
    bias = torch.arange(5.0, device=dev)
    C = _gemm(z, torch.zeros(0, 5, device=dev), bias, 3, 5, 0, 0, 0)
    assert torch.equal(C.cpu(), bias.cpu().expand(3, 5))
    base = torch.randn(1 + 37 * 19, device=dev)
    A = base[1:].view(37, 19)
    B = torch.randn(19, 23, device=dev)
    C = _gemm(A, B, None, 37, 23, 19, 0, 0)
    ref = A.cpu().double() @ B.cpu().double()
    assert (C.cpu().double() - ref).abs().max() < 1e-4
