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


@pytest.fixture
def split_products():
    prev = _lib.set_split_products(1)
    yield
    _lib.set_split_products(prev)


def _both(A, B, bias, M, N, K, lda=None, ldb=None, ta=0, tb=1):
    """C = op(A) op(B) (+bias) by the split-bf16 kernel and by the fp32 MFMA kernel
    (A B^T by default; ta=1, tb=0 for A^T B, with the workspace hsl_gemm_ws_bytes asks)."""
    dev = A.device
    out = []
    nbytes = _lib.load().hsl_gemm_ws_bytes(M, N, K)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    for on in (1, 0):
        _lib.set_split_products(on)
        C = torch.empty(M, N, device=dev)
        P = _lib.ptr
        _lib.call("hsl_gemm_f32", P(A), P(B), P(bias), P(C), M, N, K, lda or A.shape[1], ldb or B.shape[1], N,
                  ta, tb, P(ws), nbytes, _lib.stream_of(dev))
        out.append(C.cpu().double())
    _lib.set_split_products(1)
    return out


@pytest.mark.parametrize("M,N,K,pad_a,pad_b", [(4096, 4096, 256, 0, 0), (4096 + 37, 4096 + 100, 207, 0, 0),
                                               (4352, 4096, 96, 3, 1), (2048, 8192, 1024, 0, 0),
                                               (2048, 4096, 512, 0, 0), (2048 + 5, 4096 - 64, 300, 1, 0)])
def test_split_products_as_accurate_as_fp32(dev, split_products, M, N, K, pad_a, pad_b):
    """Large A B^T products (>= 256 tiles of 256x256, or of 256x128: the last two shapes)
    take the split-bf16 kernel: every
    fp32 operand is split exactly into three bf16 pieces and the six largest piece
    products are accumulated in fp32.  Against the fp64 product it must meet the fp32
    bound, and its error statistics must match those of the fp32 MFMA kernel on the
    same operands (rows sampled for the fp64 reference)."""
    print(f"split products M={M} N={N} K={K} pad=({pad_a},{pad_b})", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randn(M, K + pad_a, generator=g)
    b = torch.randn(N, K + pad_b, generator=g) * 0.1
    bias = torch.randn(N, generator=g)
    cx6, c32 = _both(a.to(dev), b.to(dev), bias.to(dev), M, N, K, K + pad_a, K + pad_b)
    assert not torch.equal(cx6, c32)  # two different kernels ran
    rows = torch.arange(0, M, 97)
    av, bv = a[rows, :K].double(), b[:, :K].double()
    ref = av @ bv.t() + bias.double()
    scale = av.abs() @ bv.abs().t() + bias.double().abs()
    ex6 = (cx6[rows] - ref).abs() / scale
    e32 = (c32[rows] - ref).abs() / scale
    print(f"  rel err x6 max {ex6.max():.3e} rms {ex6.pow(2).mean().sqrt():.3e}; "
          f"fp32 max {e32.max():.3e} rms {e32.pow(2).mean().sqrt():.3e}", flush=True)
    assert float(ex6.max()) <= 2e-6 * K ** 0.5
    assert float(ex6.pow(2).mean().sqrt()) <= 1.25 * float(e32.pow(2).mean().sqrt()) + 1e-12
    assert float(ex6.max()) <= 2.0 * float(e32.max()) + 1e-12


def test_split_products_non_finite(dev, split_products):
    """A non-finite element of A makes its row of C NaN, one of B its column (piece
    products of an infinite piece with zero pieces are NaN); finite values beyond the
    bf16 range count as non-finite.  Everything else is unaffected, and the fp32 path
    (split products off) keeps the IEEE results."""
    M, N, K = 4096, 4096, 64
    g = torch.Generator().manual_seed(5)
    a = torch.randn(M, K, generator=g)
    b = torch.rand(N, K, generator=g) + 0.5
    a[3, 5] = float("inf")
    a[700, 0] = -float("inf")
    a[1200, 9] = float("nan")
    a[2000, 1] = 3.4e38  # finite in fp32, beyond bf16
    b[17, 2] = float("inf")
    cx6, c32 = _both(a.to(dev), b.to(dev), None, M, N, K)
    bad_rows = torch.tensor([3, 700, 1200, 2000])
    for r in bad_rows.tolist():
        assert bool(torch.isnan(cx6[r]).all()), r
    assert bool(torch.isnan(cx6[:, 17]).all())
    keep = torch.ones(M, dtype=torch.bool)
    keep[bad_rows] = False
    rest = cx6[keep][:, torch.arange(N) != 17]
    assert bool(torch.isfinite(rest).all())
    ref = c32[keep][:, torch.arange(N) != 17]
    assert float(((rest - ref).abs() / (ref.abs() + 1.0)).max()) < 1e-5
    # the fp32 instruction: IEEE infinities
    assert bool(torch.isposinf(c32[3, :17]).all()) and bool(torch.isneginf(c32[700, :17]).all())
    assert bool(torch.isnan(c32[1200]).all()) and bool(torch.isinf(c32[5:10, 17]).all())
    assert torch.equal(torch.sign(c32[5:10, 17]), torch.sign(a[5:10, 2]).double())


@pytest.mark.parametrize("M,N,K,pad,ta", [(4096, 256, 65536, 0, 1), (2048, 512, 8192, 0, 1), (1000, 300, 20000, 3, 1),
                                          (65536, 256, 4096, 0, 0), (2048, 1024, 8192, 0, 0), (3000, 300, 5000, 1, 0)])
def test_split_products_weight_gradient_layout(dev, split_products, M, N, K, pad, ta):
    """C = A^T B over a long K (the weight gradients dgates^T x, K = T*B) and C = A B
    (dx = dgates W_ih, K = 4H): the split-bf16 kernel sums fp32 runs of 64 k into a second
    fp32 accumulator and splits K into planes of at most 2048 k added in fp64; against the
    fp64 product it must meet the fp32 bound and match the fp32 kernel's error (rows
    sampled)."""
    print(f"split products {'A^T B' if ta else 'A B'} M={M} N={N} K={K} pad={pad}", flush=True)
    g = torch.Generator().manual_seed(M + 3 * N + K + ta)
    if ta:
        a = torch.randn(K, M + pad, generator=g) * 0.05   # dgates-like [K, M]
    else:
        a = torch.randn(M, K + pad, generator=g) * 0.05   # dgates-like [M, K]
    b = torch.randn(K, N + pad, generator=g)              # [K, N]
    cx6, c32 = _both(a.to(dev), b.to(dev), None, M, N, K, ta=ta, tb=0)
    assert not torch.equal(cx6, c32)
    rows = torch.arange(0, M, max(1, M // 100))
    av = (a[:, rows].t() if ta else a[rows, :K]).double()
    bv = b[:, :N].double()
    ref = av @ bv
    scale = av.abs() @ bv.abs()
    ex6 = (cx6[rows] - ref).abs() / scale
    e32 = (c32[rows] - ref).abs() / scale
    print(f"  rel err x6 max {ex6.max():.3e} rms {ex6.pow(2).mean().sqrt():.3e}; "
          f"fp32 max {e32.max():.3e} rms {e32.pow(2).mean().sqrt():.3e}", flush=True)
    assert float(ex6.max()) <= 2e-6 * K ** 0.5
    assert float(ex6.pow(2).mean().sqrt()) <= 1.25 * float(e32.pow(2).mean().sqrt()) + 1e-12
    assert float(ex6.max()) <= 2.0 * float(e32.max()) + 1e-12


@pytest.mark.parametrize("layout", ["abt", "abt_narrow", "atb", "ab"])
@pytest.mark.parametrize("three_piece", ["a", "b"])
def test_split_products_exact_on_representable_sums(dev, split_products, layout, three_piece):
    """Pins the piece bookkeeping of the split-bf16 kernels by exact arithmetic.  One
    operand holds values m * 2^-16 with |m| < 2^18 (three non-zero bf16 pieces in
    general), the other +-1 (one piece), and only 32 k-values are non-zero.  Every piece
    product that is kept then enters exactly, every partial sum is a multiple of 2^-16
    below 2^7 in magnitude, which fp32 represents exactly, so the result must equal the
    exact sum bit for bit: a wrong, swapped or missing piece changes it.  The long-K
    layouts (A^T B, A B) run over K = 8192 (their size rule) with the 32 non-zero k in one
    band, which also exercises their k-splits and the fp64 sum of the planes."""
    g = torch.Generator().manual_seed(len(layout) * 7 + (three_piece == "a"))

    def fine(*shape):
        return torch.randint(-(1 << 18) + 1, 1 << 18, shape, generator=g).double() * 2.0 ** -16

    def sign(*shape):
        return torch.randint(0, 2, shape, generator=g).double() * 2 - 1

    def pair(shape_a, shape_b):
        return (fine(*shape_a), sign(*shape_b)) if three_piece == "a" else (sign(*shape_a), fine(*shape_b))

    if layout.startswith("abt"):  # C = A B^T, A [M,K], B [N,K]; narrow: 256 tiles of 256x128
        M, N, K = (4096, 4096, 32) if layout == "abt" else (2048, 4096, 32)
        a, b = pair((M, K), (N, K))
        exact, ta = a @ b.t(), 0
    else:
        M, N, K = 4096, 256, 8192
        band = torch.zeros(K, dtype=torch.double)
        band[1024:1056] = 1.0
        if layout == "atb":  # C = A^T B, A [K,M], B [K,N]
            a, b = pair((K, M), (K, N))
            a, b = a * band[:, None], b * band[:, None]
            exact, ta = a.t() @ b, 1
        else:  # C = A B, A [M,K], B [K,N]
            a, b = pair((M, K), (K, N))
            a, b = a * band[None, :], b * band[:, None]
            exact, ta = a @ b, 0
    print(f"exact sums layout={layout} three-piece operand={three_piece} M={M} N={N} K={K}", flush=True)
    cx6, c32 = _both(a.float().to(dev), b.float().to(dev), None, M, N, K, ta=ta, tb=int(layout.startswith("abt")))
    assert torch.equal(cx6, exact)
    assert torch.equal(c32, exact)
