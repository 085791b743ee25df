"""fp64 modules on the GPU (the ``*_f64`` entry points).

The reference runs fp64 modules through its torch backend (``test_cpp.py:150-165``) and
its parallel functional is dtype-generic (``_parallel.py:38-74``).  Here an fp64 module
runs fp64 kernels, so every output and gradient must match the fp64 CPU restatement
(the oracle) to fp64 rounding (rtol 1e-10, atol 1e-12: the two differ only in the order
of their additions), and torch's numerical gradient check must pass on the GPU
functionals themselves.
"""

import pytest
import torch

from conftest import lim_ratio
from oracle import hsl_oracle as O
import prlstm_amd
from prlstm_amd import functional

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-10, 1e-12


def _run(m, x, hx, wts, dev=None):
    x = (x.to(dev) if dev else x).clone().requires_grad_(True)
    if hx is not None:
        hx = tuple((t.to(dev) if dev else t).clone().requires_grad_(True) for t in hx)
    out, (h_n, c_n) = m(x, hx)
    w = [t.to(dev) if dev else t for t in wts]
    ((out * w[0]).sum() + (h_n[0] * w[1]).sum() + (c_n[0] * w[2]).sum()).backward()
    res = {"out": out, "h_n": h_n, "c_n": c_n, "dx": x.grad}
    for n, p in m.named_parameters():
        res["d" + n] = p.grad
    if hx is not None:
        res["dh0"], res["dc0"] = hx[0].grad, hx[1].grad
    return res


def _check(T, B, D, H, dev, parallel, with_hx=False, batch_first=False, seed=0, sum_atol=ATOL):
    print(f"fp64 T={T} B={B} D={D} H={H} parallel={parallel} hx={with_hx} bf={batch_first}", flush=True)
    torch.manual_seed(seed)
    ref = O.RefHeadStartLSTM(D, H, batch_first=batch_first, parallel=parallel).double()
    with torch.no_grad():
        ref.a.copy_(torch.tensor([0.3, 0.2, 0.4, 0.1], dtype=torch.float64))
    g = torch.Generator().manual_seed(seed + 1)
    shape = (B, T, D) if batch_first else (T, B, D)
    x = torch.randn(*shape, generator=g, dtype=torch.float64)
    hx = None
    if with_hx:
        hx = (0.5 * torch.randn(1, B, H, generator=g, dtype=torch.float64),
              torch.rand(1, B, H, generator=g, dtype=torch.float64))
    oshape = (B, T, H) if batch_first else (T, B, H)
    wts = tuple(torch.randn(*s, generator=g, dtype=torch.float64) for s in (oshape, (B, H), (B, H)))
    r_ref = _run(ref, x, hx, wts)
    m = prlstm_amd.HeadStartLSTM(D, H, batch_first=batch_first, parallel=parallel).double()
    m.load_state_dict(ref.state_dict())
    m = m.to(dev)
    r_gpu = _run(m, x, hx, wts, dev)
    torch.cuda.synchronize()
    for k, v in r_ref.items():
        if v is None:  # the reference's dh0/dc0 (recurrent mode returns None for them)
            continue
        assert r_gpu[k].dtype == torch.float64, k
        # parameter gradients are sums over all T*B rows: sum_atol for long ones
        ratio = lim_ratio(r_gpu[k], v, RTOL, sum_atol if k.startswith(("dweight", "dbias", "da")) else ATOL)
        print(f"  {k:16s} {ratio:.3g}x of the fp64 tolerance")
        assert ratio <= 1.0, (k, ratio)
    if with_hx and not parallel:  # dh0/dc0 against fp64 autograd of the textbook LSTM
        xb = x.transpose(0, 1).contiguous() if batch_first else x
        h0 = hx[0][0].clone().requires_grad_(True)
        c0 = hx[1][0].clone().requires_grad_(True)
        out, h, c = O.textbook_forward(xb, h0, c0, *[p.detach() for p in ref.parameters()])
        w0 = wts[0].transpose(0, 1) if batch_first else wts[0]
        ((out * w0).sum() + (h * wts[1]).sum() + (c * wts[2]).sum()).backward()
        assert lim_ratio(r_gpu["dh0"].reshape(B, H), h0.grad, RTOL, ATOL) <= 1.0
        assert lim_ratio(r_gpu["dc0"].reshape(B, H), c0.grad, RTOL, ATOL) <= 1.0
    return r_gpu


SHAPES = [(12, 3, 16, 24), (37, 5, 9, 70), (1, 1, 1, 1), (130, 2, 8, 40)]


@pytest.mark.parametrize("parallel", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_f64_matches_oracle(dev, parallel, shape):
    _check(*shape, dev, parallel)


def test_f64_config2_full_size(dev):
    """configs[2] (T256 B32 D256 H512) as an fp64 module in recurrent mode, every element
    against the fp64 oracle, with hx and a ~ (0.3, 0.2, 0.4, 0.1).  The parameter gradients
    sum 8192 rows (sqrt(K) u rms(term) rounding in any order), hence atol 1e-9 for them."""
    _check(256, 32, 256, 512, dev, False, with_hx=True, seed=21, sum_atol=1e-9)


def test_f64_parallel_multi_group_chunks(dev):
    """Parallel mode with enough channels (B*H = 65536) that the scans cut T = 70 into
    chunks of 24 steps (three checkpoint groups); the last chunk has 22 steps.

    The reference here is the linear-domain fp64 recurrence (``O.linear_scan``, pinned to
    the log-domain scan by the oracle tests) under autograd: at this size the log-domain
    form's own fp64 rounding differs from the linear form by 1.4x the 1e-10 tolerance on
    db_ih (a 4480-row column sum with cancellation), while two summation orders of the
    same dgates differ by < 0.01x."""
    T, B, D, H = 70, 64, 8, 1024
    print(f"fp64 parallel chunks T={T} B={B} D={D} H={H}", flush=True)
    torch.manual_seed(9)
    m = prlstm_amd.HeadStartLSTM(D, H, parallel=True).double()
    g = torch.Generator().manual_seed(10)
    x = torch.randn(T, B, D, generator=g, dtype=torch.float64)
    c0 = torch.rand(1, B, H, generator=g, dtype=torch.float64)
    c0[0, :, :8] = 0.0  # clamped entries of c0
    wts = tuple(torch.randn(*s, generator=g, dtype=torch.float64) for s in ((T, B, H), (B, H), (B, H)))
    xr = x.clone().requires_grad_(True)
    c0r = c0.clone().requires_grad_(True)
    w_ih = m.weight_ih_l0.detach().clone().requires_grad_(True)
    b_ih = m.bias_ih_l0.detach().clone().requires_grad_(True)
    gi, gf, gg, go = torch.sigmoid(torch.nn.functional.linear(xr, w_ih, b_ih)).chunk(4, dim=-1)
    c = O.linear_scan(gf, gi * gg, c0r[0])
    out = go * torch.tanh(c)
    ((out * wts[0]).sum() + (out[-1] * wts[1]).sum() + (c[-1] * wts[2]).sum()).backward()
    ref = {"out": out, "h_n": out[-1:], "c_n": c[-1:], "dx": xr.grad, "dweight_ih_l0": w_ih.grad,
           "dbias_ih_l0": b_ih.grad, "dc0": c0r.grad}
    r_gpu = _run(m.to(dev), x, (torch.zeros(1, B, H, dtype=torch.float64), c0), wts, dev)
    torch.cuda.synchronize()
    for k, v in ref.items():
        ratio = lim_ratio(r_gpu[k], v, RTOL, ATOL)
        print(f"  {k:16s} {ratio:.3g}x of the fp64 tolerance")
        assert ratio <= 1.0, (k, ratio)


@pytest.mark.parametrize("parallel", [False, True])
def test_f64_hx_and_batch_first(dev, parallel):
    _check(20, 4, 12, 36, dev, parallel, with_hx=True, batch_first=True, seed=3)


@pytest.mark.parametrize("parallel", [False, True])
def test_f64_deterministic(dev, parallel):
    a = _check(40, 3, 16, 32, dev, parallel, seed=5)
    b = _check(40, 3, 16, 32, dev, parallel, seed=5)
    for k in a:
        if a[k] is not None:
            assert torch.equal(a[k], b[k]), k


def test_f64_clamps_active(dev):
    """Parallel mode with gate pre-activations large enough that sigmoid(f) and i*g fall
    below eps = 1e-6 and c0 entries below eps: the clamps and their gradient masks."""
    T, B, D, H = 24, 3, 6, 20
    torch.manual_seed(7)
    ref = O.RefHeadStartLSTM(D, H, parallel=True).double()
    with torch.no_grad():
        ref.weight_ih_l0.mul_(12.0)
        ref.bias_ih_l0.mul_(12.0)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(T, B, D, generator=g, dtype=torch.float64)
    c0 = torch.rand(1, B, H, generator=g, dtype=torch.float64)
    c0[0, 0, :5] = 0.0
    c0[0, 1, :5] = -2.0
    c0[0, 2, :5] = 1e-7
    hx = (torch.zeros(1, B, H, dtype=torch.float64), c0)
    wts = tuple(torch.randn(*s, generator=g, dtype=torch.float64) for s in ((T, B, H), (B, H), (B, H)))
    r_ref = _run(ref, x, hx, wts)
    m = prlstm_amd.HeadStartLSTM(D, H, parallel=True).double()
    m.load_state_dict(ref.state_dict())
    r_gpu = _run(m.to(dev), x, hx, wts, dev)
    for k, v in r_ref.items():
        if v is not None:
            assert lim_ratio(r_gpu[k], v, 1e-9, 1e-12) <= 1.0, k


@pytest.mark.parametrize("parallel", [False, True])
def test_f64_gradcheck(dev, parallel):
    """torch.autograd.gradcheck of the GPU functional (central differences against the
    analytical backward) for every differentiable input."""
    T, B, D, H = 4, 2, 3, 4
    torch.manual_seed(11)
    f64 = dict(device=dev, dtype=torch.float64)
    x = torch.randn(T, B, D, **f64, requires_grad=True)
    h0 = (0.5 * torch.randn(B, H, **f64)).requires_grad_(not parallel)
    c0 = (0.5 + 0.5 * torch.rand(B, H, **f64)).requires_grad_(True)
    w_ih = (0.5 * torch.randn(4 * H, D, **f64)).requires_grad_(True)
    w_hh = (0.5 * torch.randn(4 * H, H, **f64)).requires_grad_(not parallel)
    b_ih = (0.5 * torch.randn(4 * H, **f64)).requires_grad_(True)
    b_hh = (0.5 * torch.randn(4 * H, **f64)).requires_grad_(not parallel)
    a = torch.tensor([0.3, 0.2, 0.4, 0.1], **f64).requires_grad_(not parallel)
    fn = functional.headstartlstm_parallel if parallel else functional.headstartlstm_recurrent
    assert torch.autograd.gradcheck(lambda *args: fn(*args), (x, h0, c0, w_ih, w_hh, b_ih, b_hh, a),
                                    eps=1e-6, atol=1e-7, rtol=1e-5)


def test_f64_config4_full_size(dev):
    """configs[4] (T4096 B16 D256 H1024) as an fp64 module: the full step (16 scan chunks
    of 256 steps, the projection and dW_ih on split K over T*B = 65536 rows) against fp64
    autograd of the linear-domain recurrence (``O.linear_scan``) on the CPU, every element
    of every output and gradient.  dW_ih and db_ih are sums of 65536 products, whose
    rounding in any order is about sqrt(K) u rms(term) ~ 1e-12, hence atol 1e-9 for them;
    the other outputs keep atol 1e-12."""
    T, B, D, H = 4096, 16, 256, 1024
    print(f"fp64 configs[4] T={T} B={B} D={D} H={H}", flush=True)
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(D, H, a_init=0.0, parallel=True).double()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(T, B, D, generator=g, dtype=torch.float64)
    c0 = torch.rand(1, B, H, generator=g, dtype=torch.float64)
    wts = tuple(torch.randn(*s, generator=g, dtype=torch.float64) for s in ((T, B, H), (B, H), (B, H)))
    xr = x.clone().requires_grad_(True)
    c0r = c0.clone().requires_grad_(True)
    w_ih = m.weight_ih_l0.detach().clone().requires_grad_(True)
    b_ih = m.bias_ih_l0.detach().clone().requires_grad_(True)
    gi, gf, gg, go = torch.sigmoid(torch.nn.functional.linear(xr, w_ih, b_ih)).chunk(4, dim=-1)
    c = O.linear_scan(gf, gi * gg, c0r[0])
    out = go * torch.tanh(c)
    ((out * wts[0]).sum() + (out[-1] * wts[1]).sum() + (c[-1] * wts[2]).sum()).backward()
    ref = {"out": out, "h_n": out[-1:], "c_n": c[-1:], "dx": xr.grad, "dweight_ih_l0": w_ih.grad,
           "dbias_ih_l0": b_ih.grad, "dc0": c0r.grad}
    del gi, gf, gg, go, c
    r_gpu = _run(m.to(dev), x, (torch.zeros(1, B, H, dtype=torch.float64), c0), wts, dev)
    torch.cuda.synchronize()
    for k, v in ref.items():
        atol = 1e-9 if k in ("dweight_ih_l0", "dbias_ih_l0") else ATOL
        ratio = lim_ratio(r_gpu[k], v, RTOL, atol)
        print(f"  {k:16s} {ratio:.3g}x of the fp64 tolerance", flush=True)
        assert ratio <= 1.0, (k, ratio)
