"""bf16 / fp16 modules: inputs and parameters in half precision, fp32 accumulation.

The reference's tests tabulate a bf16 tolerance of 1e-2 (``test_parallel.py:22``)
for modules moved with ``.to(device, dtype)`` (``:37-38``) but never run it.  Here a
half-precision module is widened to fp32 at the functional, computed by the same
fp32 kernels, and rounded back, so two checks pin it:
* exactness: outputs and gradients equal the fp32 module's on the widened operands,
  rounded to the half dtype (any extra rounding inside would break this);
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
    for name, a16, a32 in [("out", out16, out32), ("h_n", h16, h32), ("c_n", c16, c32), ("dx", dx16, dx32)]:
        assert a16.dtype == dtype, name
        assert torch.equal(a16, a32.to(dtype)), name
    for n in g32:
        if g32[n] is None:
            assert g16[n] is None, n
        else:
            assert g16[n].dtype == dtype, n
            assert torch.equal(g16[n], g32[n].to(dtype)), n


def test_bf16_module_within_reference_tolerance(dev):
    """The reference's bf16 bar (max |diff| < 1e-2) against the fp64 oracle."""
    T, B, D, H = 32, 4, 16, 24
    torch.manual_seed(0)
    m16 = prlstm_amd.HeadStartLSTM(D, H).to(dev, torch.bfloat16)
    x16 = torch.randn(T, B, D, device=dev).to(torch.bfloat16)
    out16, (h16, c16) = m16(x16)
    ref = O.RefHeadStartLSTM(D, H).double()
    with torch.no_grad():
        for pr, p16 in zip(ref.parameters(), m16.parameters()):
            pr.copy_(p16.double().cpu())
    out64, (h64, c64) = ref(x16.double().cpu())
    for name, got, want in [("out", out16, out64), ("h_n", h16, h64), ("c_n", c16, c64)]:
        d = (got.double().cpu() - want).abs().max().item()
        print(f"  {name} max |bf16 - fp64| = {d:.3e}", flush=True)
        assert d < 1e-2, name
