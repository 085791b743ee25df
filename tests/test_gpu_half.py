"""bf16 / fp16 modules: inputs and parameters in half precision, fp32 accumulation.

The reference's tests tabulate a bf16 tolerance of 1e-2 (``test_parallel.py:22``)
for modules moved with ``.to(device, dtype)`` (``:37-38``) but never run it.  Here a
half-precision module is computed by the fp32 kernels on widened operands and rounded
back; in parallel mode its input projection runs on 16-bit MFMA instead (products of
16-bit values are exact in fp32, only the summation order differs).  The checks:
* recurrent mode: outputs and gradients equal the fp32 module's on the widened
  operands, rounded to the half dtype (any extra rounding inside would break this);
* parallel mode: the same within one unit in the last place of the half dtype, and
  bitwise for nearly every element (the fp32 sums differ only in their order);
* the reference's bf16 tolerance against the fp64 oracle on the same operands.
"""

import pytest
import torch

from oracle import hsl_oracle as O
import prlstm_amd

pytestmark = pytest.mark.gpu


def _step(m, x):
    m.zero_grad(set_to_none=True)
    x = x.clone().requires_grad_(True)
    out, (h_n, c_n) = m(x)
    ((out.float() * 0.5).sum() + h_n.float().sum() + c_n.float().sum()).backward()
    grads = {n: (None if p.grad is None else p.grad) for n, p in m.named_parameters()}
    return out, h_n, c_n, x.grad, grads


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("parallel", [False, True])
def test_half_module_equals_rounded_fp32(dev, dtype, parallel):
    T, B, D, H = 12, 3, 16, 24
    print(f"half {dtype} parallel={parallel}", flush=True)
    torch.manual_seed(0)
    m16 = prlstm_amd.HeadStartLSTM(D, H, parallel=parallel).to(dev, dtype)
    with torch.no_grad():
        m16.a.fill_(0.25)
    m32 = prlstm_amd.HeadStartLSTM(D, H, parallel=parallel).to(dev)
    with torch.no_grad():
        for p32, p16 in zip(m32.parameters(), m16.parameters()):
            p32.copy_(p16.float())
    x16 = torch.randn(T, B, D, device=dev).to(dtype)
    out16, h16, c16, dx16, g16 = _step(m16, x16)
    out32, h32, c32, dx32, g32 = _step(m32, x16.float())
    def same(name, a16, a32):
        r = a32.to(dtype)
        if not parallel:
            assert torch.equal(a16, r), name
            return
        ulp = (r.float().abs() * (2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10)).clamp_min(1e-30)
        diff = (a16.float() - r.float()).abs()
        assert bool((diff <= ulp * 1.0001 + 1e-30).all()), (name, float((diff / ulp).max()))
        assert float((a16 == r).float().mean()) >= 0.97, name

    for name, a16, a32 in [("out", out16, out32), ("h_n", h16, h32), ("c_n", c16, c32), ("dx", dx16, dx32)]:
        assert a16.dtype == dtype, name
        same(name, a16, a32)
    for n in g32:
        if g32[n] is None:
            assert g16[n] is None, n
        else:
            assert g16[n].dtype == dtype, n
            same(n, g16[n], g32[n])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("parallel", [False, True])
def test_half_module_within_reference_tolerance(dev, parallel, dtype):
    """Against the fp64 oracle on the same (16-bit) operands.  bf16: the reference's bar,
    max |diff| < 1e-2 (test_parallel.py:22-24).  fp16 (no bar in the reference): 1e-3,
    the same bar scaled to fp16's 3 more significand bits (its half-ulp at 1 is 4.9e-4).
    Gradients (x and every parameter the mode trains) by the same bar, relative to the
    largest magnitude of each gradient (they are sums over T*B terms)."""
    T, B, D, H = 32, 4, 16, 24
    bar = 1e-2 if dtype == torch.bfloat16 else 1e-3
    print(f"half {dtype} parallel={parallel} vs fp64 oracle", flush=True)
    torch.manual_seed(0)
    m16 = prlstm_amd.HeadStartLSTM(D, H, parallel=parallel).to(dev, dtype)
    with torch.no_grad():
        m16.a.fill_(0.25)
    x16 = torch.randn(T, B, D, device=dev).to(dtype).requires_grad_(True)
    out16, (h16, c16) = m16(x16)
    out16.float().sum().backward()
    ref = O.RefHeadStartLSTM(D, H, parallel=parallel).double()
    with torch.no_grad():
        for pr, p16 in zip(ref.parameters(), m16.parameters()):
            pr.copy_(p16.double().cpu())
    x64 = x16.detach().double().cpu().requires_grad_(True)
    out64, (h64, c64) = ref(x64)
    out64.sum().backward()
    for name, got, want in [("out", out16, out64), ("h_n", h16, h64), ("c_n", c16, c64)]:
        d = (got.double().cpu() - want).abs().max().item()
        print(f"  {name} max |{dtype} - fp64| = {d:.3e}", flush=True)
        assert d < bar, name
    grads = [("dx", x16.grad, x64.grad)]
    grads += [("d" + n, p.grad, q.grad) for (n, p), q in zip(m16.named_parameters(), ref.parameters())]
    for name, got, want in grads:
        if want is None:
            assert got is None, name
            continue
        assert got.dtype == dtype, name
        d = (got.double().cpu() - want).abs().max().item() / max(want.abs().max().item(), 1e-30)
        print(f"  {name} max |{dtype} - fp64| / max|fp64| = {d:.3e}", flush=True)
        assert d < bar, name


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (5, 7, 3), (33, 65, 17), (128, 128, 64), (300, 200, 136),
                                   (256, 384, 256), (4096, 1024, 256)])
def test_gemm_b16_matches_fp64(dev, fmt, M, N, K):
    """hsl_gemm_b16 (C = A B^T + bias, 16-bit A and B) against the fp64 product of the
    widened operands: every product is exact in fp32, so only fp32 summation error
    (bounded by 2e-6 sqrt(K) sum|a b|) remains."""
    dt = torch.bfloat16 if fmt == 0 else torch.float16
    print(f"gemm_b16 fmt={fmt} M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 13 + N * 5 + K + fmt)
    a = torch.randn(M, K, generator=g).to(dt)
    b = torch.randn(N, K, generator=g).to(dt)
    bias = torch.randn(N, generator=g)
    C = torch.empty(M, N, device=dev)
    from prlstm_amd import _lib
    P = _lib.ptr
    A, Bm = a.to(dev), b.to(dev)
    _lib.call("hsl_gemm_b16", P(A), P(Bm), P(bias.to(dev)), P(C), M, N, K, K, K, N, fmt, _lib.stream_of(dev))
    ref = a.double() @ b.double().t() + bias.double()
    scale = a.double().abs() @ b.double().abs().t() + bias.double().abs()
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= 2e-6 * max(K, 1) ** 0.5 * scale + 1e-30).all()), float((err / scale).max())


def test_gemm_b16_unaligned_rows(dev):
    """Odd leading dimensions take the masked (element-wise) loads."""
    M, N, K = 70, 90, 37
    g = torch.Generator().manual_seed(7)
    a = torch.randn(M, K + 3, generator=g).to(torch.bfloat16)
    b = torch.randn(N, K + 5, generator=g).to(torch.bfloat16)
    C = torch.empty(M, N, device=dev)
    from prlstm_amd import _lib
    P = _lib.ptr
    A, Bm = a.to(dev), b.to(dev)
    _lib.call("hsl_gemm_b16", P(A), P(Bm), None, P(C), M, N, K, K + 3, K + 5, N, 0, _lib.stream_of(dev))
    ref = a[:, :K].double() @ b[:, :K].double().t()
    scale = a[:, :K].double().abs() @ b[:, :K].double().abs().t()
    err = (C.cpu().double() - ref).abs()
    assert bool((err <= 2e-6 * K ** 0.5 * scale + 1e-30).all())


@pytest.mark.parametrize("fmt", [0, 1])
@pytest.mark.parametrize("T,B,D,H", [(32, 4, 16, 24), (4096, 16, 256, 1024)])
def test_parallel_backward_16bit_operands_equal_widened(dev, fmt, T, B, D, H):
    """hsl_par_bwd_b16 reads the 16-bit x and W_ih itself: a bf16 value is one bf16 piece,
    so the split-product kernel issues three products per k-step instead of six (at
    configs[4] size), and otherwise the operand is widened into the workspace.  Either way
    the gradients must equal hsl_par_bwd's on the widened operands bit for bit (the six
    products' extra terms are exact zeros added in the same order).  hsl_par_fwd_b16 writes
    out in the 16-bit format: the fp32 scan output of the same gates (hsl_scan_fwd)
    rounded to nearest even, bit for bit; the backward reads the 16-bit dout."""
    dt = torch.bfloat16 if fmt == 0 else torch.float16
    print(f"par bwd 16-bit fmt={fmt} T={T} B={B} D={D} H={H}", flush=True)
    from prlstm_amd import _lib
    P, s = _lib.ptr, _lib.stream_of(dev)
    g = torch.Generator().manual_seed(T + D)
    x16 = torch.randn(T, B, D, generator=g).to(dt).to(dev)
    w16 = (torch.randn(4 * H, D, generator=g) * 0.05).to(dt).to(dev)
    b_ih = (torch.randn(4 * H, generator=g) * 0.05).to(dev)
    c0 = (torch.randn(B, H, generator=g) * 0.5).to(dev)
    gates = torch.empty(T, B, 4 * H, device=dev)
    out = torch.empty(T, B, H, dtype=dt, device=dev)
    c_ck = torch.empty(_lib.load().hsl_scan_ck_rows(T), B, H, device=dev)
    _lib.call("hsl_par_fwd_b16", P(x16), P(c0), P(w16), P(b_ih), 1e-6, P(gates), P(out), P(c_ck),
              T, B, D, H, fmt, s)
    out32 = torch.empty(T, B, H, device=dev)
    ck32 = torch.empty_like(c_ck)
    _lib.call("hsl_scan_fwd", P(gates), P(c0), 1e-6, P(out32), P(ck32), T, B, H, s)
    torch.cuda.synchronize()
    assert torch.equal(out, out32.to(dt))
    assert torch.equal(c_ck, ck32)
    dout16 = torch.randn(T, B, H, generator=g).to(dt).to(dev)
    dout32 = dout16.float()
    dh_n = torch.randn(B, H, generator=g).to(dev)
    dc_n = torch.randn(B, H, generator=g).to(dev)
    res = []
    for widened in (False, True):
        dx = torch.empty(T, B, D, device=dev)
        dw = torch.empty(4 * H, D, device=dev)
        db = torch.empty(4 * H, device=dev)
        dc0 = torch.empty(B, H, device=dev)
        if widened:
            xw, ww = x16.float(), w16.float()
            n = _lib.load().hsl_par_bwd_ws_bytes(T, B, D, H)
            ws = torch.empty(n, dtype=torch.uint8, device=dev)
            _lib.call("hsl_par_bwd", P(dout32), P(dh_n), P(dc_n), P(xw), P(c0), P(gates), P(c_ck), P(ww), 1e-6,
                      P(dx), P(dw), P(db), P(dc0), P(ws), n, T, B, D, H, s)
        else:
            n = _lib.load().hsl_par_bwd_b16_ws_bytes(T, B, D, H)
            ws = torch.empty(n, dtype=torch.uint8, device=dev)
            _lib.call("hsl_par_bwd_b16", P(dout16), P(dh_n), P(dc_n), P(x16), P(c0), P(gates), P(c_ck), P(w16),
                      1e-6, P(dx), P(dw), P(db), P(dc0), P(ws), n, T, B, D, H, fmt, s)
        torch.cuda.synchronize()
        res.append((dx.clone(), dw.clone(), db.clone(), dc0.clone()))
    for name, a, b in zip(("dx", "dW_ih", "db_ih", "dc0"), res[0], res[1]):
        assert torch.isfinite(a).all(), name
        assert torch.equal(a, b), (name, float((a - b).abs().max()))
