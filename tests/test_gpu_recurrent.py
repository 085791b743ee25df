"""Recurrent mode on the GPU vs the CPU restatement of the reference torch backend.

Every output and gradient must be within rtol 1e-4 / atol 1e-5 of the fp32 CPU
restatement (``assert_parity``, with the fp64 tie-break where the CPU's own
rounding reaches the tolerance).  Both recurrent paths are checked: the
persistent kernels (path 2) and the one-launch-per-step kernels (path 1).
"""

import pytest
import torch

from conftest import assert_parity
from oracle import hsl_oracle as O
import prlstm_amd
from prlstm_amd import functional

pytestmark = pytest.mark.gpu

NAMES = ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0", "a"]


@pytest.fixture(autouse=True)
def _debug():
    functional.debug_checks(True)
    yield
    functional.debug_checks(False)
    prlstm_amd.set_recurrent_path(0)
    prlstm_amd.set_exchange_scope(0)


def _run_ref(m, x, hx, wts):
    x = x.clone().requires_grad_(True)
    if hx is not None:
        hx = tuple(t.clone().requires_grad_(True) for t in hx)
    out, (h_n, c_n) = m(x, hx)
    loss = (out * wts[0]).sum() + (h_n[0] * wts[1]).sum() + (c_n[0] * wts[2]).sum()
    loss.backward()
    res = {"out": out, "h_n": h_n, "c_n": c_n, "dx": x.grad}
    for n, p in m.named_parameters():
        res["d" + n] = p.grad
    return res


def _run_gpu(m, x, hx, wts, dev):
    x = x.to(dev).requires_grad_(True)
    if hx is not None:
        hx = tuple(t.to(dev).requires_grad_(True) for t in hx)
    out, (h_n, c_n) = m(x, hx)
    fwd_path = prlstm_amd.last_recurrent_path()
    w = [t.to(dev) for t in wts]
    loss = (out * w[0]).sum() + (h_n[0] * w[1]).sum() + (c_n[0] * w[2]).sum()
    loss.backward()
    res = {"out": out, "h_n": h_n, "c_n": c_n, "dx": x.grad}
    for n, p in m.named_parameters():
        res["d" + n] = p.grad
    if hx is not None:
        res["dh0"], res["dc0"] = hx[0].grad, hx[1].grad
    return res, fwd_path


def check(T, B, D, H, dev, path, a=None, seed=0, with_hx=False, batch_first=False, fwd_path=None):
    """path: 1 or 2 forces that path (and checks the backward took it); 0 lets the library
    choose.  fwd_path: the path the forward must have taken (3 = the W_hh-resident forward
    for large H)."""
    print(f"recurrent T={T} B={B} D={D} H={H} path={path} a={a} hx={with_hx} bf={batch_first}",
          flush=True)
    torch.manual_seed(seed)
    ref = O.RefHeadStartLSTM(D, H, batch_first=batch_first)
    if a is not None:
        with torch.no_grad():
            ref.a.copy_(torch.as_tensor(a, dtype=torch.float32))
    shape = (B, T, D) if batch_first else (T, B, D)
    x = torch.randn(*shape)
    g = torch.Generator().manual_seed(seed + 1)
    hx = None
    if with_hx:
        hx = (0.5 * torch.randn(1, B, H, generator=g), 0.5 * torch.randn(1, B, H, generator=g))
    oshape = (B, T, H) if batch_first else (T, B, H)
    wts = (torch.randn(*oshape, generator=g), torch.randn(B, H, generator=g), torch.randn(B, H, generator=g))

    r32 = _run_ref(ref, x, hx, wts)
    ref64 = O.RefHeadStartLSTM(D, H, batch_first=batch_first).double()
    ref64.load_state_dict(ref.state_dict())
    r64 = _run_ref(ref64, x.double(), None if hx is None else tuple(t.double() for t in hx),
                   tuple(t.double() for t in wts))

    m = prlstm_amd.HeadStartLSTM(D, H, batch_first=batch_first)
    m.load_state_dict(ref.state_dict())
    m = m.to(dev)
    prlstm_amd.set_recurrent_path(path)
    rg, fp = _run_gpu(m, x, hx, wts, dev)
    if path:
        assert prlstm_amd.last_recurrent_path() == path
    if fwd_path is not None:
        assert fp == fwd_path, (fp, fwd_path)
    torch.cuda.synchronize()
    for k in r32:
        assert_parity(k, rg[k], r32[k], r64[k])
    if with_hx:  # the reference torch backend returns None here; compare with fp64 autograd
        t64 = _textbook_hx_grads(ref64, x.double(), tuple(t.double() for t in hx),
                                 tuple(t.double() for t in wts), batch_first)
        for k in ("dh0", "dc0"):
            assert_parity(k, rg[k].reshape(t64[k].shape), t64[k].float(), t64[k])
    return rg


def _textbook_hx_grads(m, x, hx, wts, batch_first):
    if batch_first:
        x = x.transpose(0, 1).contiguous()
    h0 = hx[0][0].clone().requires_grad_(True)
    c0 = hx[1][0].clone().requires_grad_(True)
    out, h, c = O.textbook_forward(x, h0, c0, *[p.detach() for p in m.parameters()])
    w0 = wts[0].transpose(0, 1) if batch_first else wts[0]
    ((out * w0).sum() + (h * wts[1]).sum() + (c * wts[2]).sum()).backward()
    return {"dh0": h0.grad, "dc0": c0.grad}


SMALL = [(10, 4, 16, 24), (8, 3, 8, 12), (12, 4, 8, 12), (1, 1, 1, 1), (5, 7, 33, 65)]


@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("shape", SMALL)
def test_small_shapes(dev, path, shape):
    check(*shape, dev, path)


@pytest.mark.parametrize("path", [1, 2])
def test_nonlinear_a_hx_batch_first(dev, path):
    check(9, 5, 12, 40, dev, path, a=[0.9, 0.3, 1.2, 0.6], with_hx=True)
    check(7, 6, 10, 20, dev, path, a=[0.5, 0.5, 0.5, 0.5], batch_first=True, seed=3)


@pytest.mark.parametrize("path", [1, 2])
def test_config0(dev, path):
    """T32 B16 D64 H128, a=1e-4."""
    check(32, 16, 64, 128, dev, path)


@pytest.mark.parametrize("path", [1, 2])
def test_config1(dev, path):
    """configs[1] recurrent: T128 B32 D256 H256."""
    check(128, 32, 256, 256, dev, path)


def test_config2_headline(dev):
    """T256 B32 D256 H512 (persistent path, as benchmarked)."""
    check(256, 32, 256, 512, dev, 2)


@pytest.mark.parametrize("shape", [(12, 5, 16, 40), (128, 32, 256, 256)])
def test_device_scope_exchange(dev, shape):
    """The persistent kernels' device-scope hand-off (used when a batch group spans XCDs)."""
    prlstm_amd.set_exchange_scope(1)
    check(*shape, dev, 2, a=[0.6, 0.2, 0.9, 0.4])


def test_config2_nonlinear_a(dev):
    """configs[2] variant: a ~ U(0, 0.5) drawn right after init."""
    torch.manual_seed(0)
    O.RefHeadStartLSTM(256, 512)
    a = torch.rand(4) * 0.5
    check(256, 32, 256, 512, dev, 2, a=a.tolist())


def test_per_step_split_products(dev):
    """Per-step path with split-K products in both directions (64 output tiles of the
    forward product, 16 of the backward one), nonlinear a and initial states."""
    check(10, 8, 64, 512, dev, 1, a=[0.4, 0.1, 0.3, 0.2], with_hx=True)


def test_config3_large_hidden(dev):
    """T64 B32 D1024 H2048 on the one-launch-per-step path."""
    check(64, 32, 1024, 2048, dev, 1)


def test_config3_wide_forward(dev):
    """configs[3] with the automatic path: forward and backward hold W_hh (64 MiB) in the
    registers of 256 workgroups (rec_fwd_wide / rec_bwd_wide, path 3)."""
    check(64, 32, 1024, 2048, dev, 0, fwd_path=3)
    assert prlstm_amd.last_recurrent_path() == 3


def test_published_h1024_shape(dev):
    """(T64, B32, D512, H1024): the reference's published shape between configs[2] and
    configs[3] (README.md:78), on the W_hh-resident kernels for H = 1024 (path 3)."""
    check(64, 32, 512, 1024, dev, 0, fwd_path=3)
    assert prlstm_amd.last_recurrent_path() == 3


def test_h1024_on_the_per_step_path(dev):
    """The same shape on the one-launch-per-step path, which the wide kernels replace."""
    check(64, 32, 512, 1024, dev, 1)


@pytest.mark.parametrize("H", [1024, 2048])
@pytest.mark.parametrize("scope", [0, 1])
@pytest.mark.parametrize("B", [20, 12])
def test_wide_forward_partial_batch_hx(dev, scope, H, B):
    """The wide kernels (both widths) with B < 32, h0/c0 given, a ~ U(0, 0.5), and with
    device-scope stores for the partial exchange (scope 1).  The batch runs as two chains of
    16 rows: B = 20 leaves 12 rows of the second chain absent, B = 12 runs one chain only."""
    prlstm_amd.set_exchange_scope(scope)
    check(6, B, 64, H, dev, 0, a=[0.3, 0.5, 0.1, 0.2], with_hx=True, fwd_path=3)
    assert prlstm_amd.last_recurrent_path() == 3


@pytest.mark.parametrize("H", [1024, 2048])
@pytest.mark.parametrize("T,B", [(1, 32), (2, 17), (3, 1), (3, 16), (3, 31)])
def test_wide_short_sequences(dev, T, B, H):
    """Edge cases of the wide kernels' chain schedule: one step (the second chain's first and
    last iterations coincide), a second chain of a single batch row, one batch row in all,
    exactly one full chain, and a second chain one row short."""
    check(T, B, 64, H, dev, 0, a=[0.3, 0.5, 0.1, 0.2], fwd_path=3)
    assert prlstm_amd.last_recurrent_path() == 3


def test_sgd_training_step(dev):
    """test_cpp.py:110-147: one SGD step (MSE loss), updated parameters agree."""
    T, B, D, H, lr = 12, 4, 8, 12, 1e-2
    torch.manual_seed(0)
    ref = O.RefHeadStartLSTM(D, H)
    m = prlstm_amd.HeadStartLSTM(D, H)
    m.load_state_dict(ref.state_dict())
    m = m.to(dev)
    x = torch.randn(T, B, D)
    target = torch.randn(T, B, H)
    for mod, xx, tt in ((ref, x, target), (m, x.to(dev), target.to(dev))):
        opt = torch.optim.SGD(mod.parameters(), lr=lr)
        opt.zero_grad()
        out, _ = mod(xx)
        ((out - tt) ** 2).mean().backward()
        opt.step()
    for (n, p), q in zip(m.named_parameters(), ref.parameters()):
        assert (p.detach().cpu() - q.detach()).abs().max() < 1e-5, n


@pytest.mark.parametrize("split", [True, False])
def test_long_sequence_persistent(dev, split):
    """T=2048 on the persistent kernels: the fused weight gradients keep at most 8 fp32
    partial planes per batch group, so each plane then spans 256 steps: 32 windows of six
    32-term bf16 piece products per running sum (split products on), or 1024 single fp32
    products (split products off), the longest running sums the backward makes."""
    prlstm_amd.set_split_products(split)
    try:
        check(2048, 4, 32, 512, dev, 2, a=[0.3, 0.2, 0.4, 0.1])
    finally:
        prlstm_amd.set_split_products(True)


def test_repeated_calls_are_deterministic(dev):
    """Persistent kernels exchange data between workgroups; repeat runs must agree bit for bit."""
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(64, 128).to(dev)
    with torch.no_grad():
        m.a.fill_(0.7)
    x = torch.randn(40, 16, 64, device=dev)
    outs = []
    for _ in range(5):
        out, _ = m(x)
        outs.append(out.detach().clone())
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("mode", ["rec1", "rec2", "par"])
def test_null_states_equal_explicit_zeros(dev, mode):
    """hx=None and an unused h_n/c_n reach the kernels as NULL pointers, read as zeros.
    The result must equal, bit for bit, the run with explicit zero states and a loss that
    touches h_n/c_n with weight zero (zero tensors passed instead of NULL)."""
    T, B, D, H = 20, 6, 16, 40
    print(f"null states {mode}", flush=True)
    if mode != "par":
        prlstm_amd.set_recurrent_path(1 if mode == "rec1" else 2)
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(D, H, parallel=(mode == "par")).to(dev)
    with torch.no_grad():
        m.a.fill_(0.6)
        m.bias_ih_l0.normal_()
    x = torch.randn(T, B, D, device=dev)
    w = torch.randn(T, B, H, device=dev)
    runs = []
    for explicit in (False, True):
        m.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_(True)
        if explicit:
            hx = (torch.zeros(1, B, H, device=dev), torch.zeros(1, B, H, device=dev))
            out, (h_n, c_n) = m(xx, hx)
            loss = (out * w).sum() + (h_n * 0).sum() + (c_n * 0).sum()
        else:
            out, (h_n, c_n) = m(xx)
            loss = (out * w).sum()
        loss.backward()
        res = {"out": out, "h_n": h_n, "c_n": c_n, "dx": xx.grad}
        res.update({n: p.grad for n, p in m.named_parameters()})
        runs.append(res)
    for k, v in runs[0].items():
        if v is None:
            assert runs[1][k] is None, k
        else:
            assert torch.equal(v, runs[1][k]), k


@pytest.mark.parametrize("split", [True, False])
@pytest.mark.parametrize("shape,fused", [((12, 5, 16, 40), 2), ((12, 5, 300, 40), 1), ((130, 6, 32, 72), 2),
                                         ((300, 6, 32, 72), 2)])
def test_fused_weight_gradients(dev, shape, fused, split):
    """The persistent backward accumulates dW_hh (and dW_ih when D <= 256) itself, on split
    bf16 products over 8-step windows (split products on) or on the fp32 instruction; the
    parity bar is the same as for the separate GEMMs.  (130 steps: two dW_hh planes with
    the fp32 products; 300 steps: two planes either way and a last window of 4 steps.)"""
    prlstm_amd.set_split_products(split)
    try:
        check(*shape, dev, 2, a=[0.4, 0.3, 0.2, 0.1])
        assert prlstm_amd._lib.last_backward_fused() == fused
    finally:
        prlstm_amd.set_split_products(True)


def test_workspaces_sized_by_path(dev):
    """The workspace queries plan the path on the device: the fused persistent forward needs
    no [T,B,4H] input-gate buffer, and a backward without dx (store_dg=0) no dgates buffer."""
    lib = prlstm_amd._lib.load()
    T, B, D, H = 256, 32, 256, 512
    gates = T * B * 4 * H * 4
    assert lib.hsl_rec_fwd_ws_bytes(T, B, D, H) < 1 << 20
    with_dx = lib.hsl_rec_bwd_ws_bytes_for(T, B, D, H, 1)
    assert with_dx == lib.hsl_rec_bwd_ws_bytes(T, B, D, H)
    assert with_dx - lib.hsl_rec_bwd_ws_bytes_for(T, B, D, H, 0) >= gates
    # configs[3] runs one launch per step: its forward needs the input-gate buffer
    assert lib.hsl_rec_fwd_ws_bytes(64, 32, 1024, 2048) >= 64 * 32 * 4 * 2048 * 4
