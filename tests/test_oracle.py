"""Pins the CPU oracle (oracle/hsl_oracle.py) before it is trusted as the checker.

The reference ships no stored vectors (its tests compute their oracles at run
time), so each oracle function is pinned by something independent of its own
formula:

* ref_init_params      -- torch's nn.LSTM draws the same four U(+-1/sqrt(H))
                          tensors in the same order: bitwise equal for a seed.
* RecurrentRefFn fwd   -- the reference's own step-by-step oracle
                          (tests/test_cpp.py:25-48, ``textbook_forward``) and a
                          scalar closed form at T=1 / T=2 written with math.*.
* RecurrentRefFn bwd   -- fp64 autograd of the textbook loop (test_cpp.py:75-107
                          in fp64, tol 1e-10) and torch.autograd.gradcheck
                          (finite differences).
* heinsen_scan         -- the linear recurrence it solves in closed form
                          (``linear_scan``) and, at T<=4, the explicit product
                          formula c_t = F_t (c0~ + sum_s b~_s / F_s).
* parallel_forward     -- a=0 equivalence with the recurrent path
                          (test_parallel.py:47-60, :84-122) and the divergence
                          sweep (test_parallel.py:63-81); its backward by gradcheck.
* RefHeadStartLSTM     -- batch_first and hx plumbing against batch rows run one
                          at a time (B=1, time-major, (B,H) state): no transpose
                          shared with the code under test.
* The last test plants mistakes in copies of the oracle and checks that the
  pins above catch them.
"""

import math

import pytest
import torch
import torch.nn as nn

from oracle import hsl_oracle as O

torch.set_num_threads(min(8, torch.get_num_threads()))


def _model(D, H, seed=0, a=None, dtype=torch.float64, parallel=False):
    torch.manual_seed(seed)
    m = O.RefHeadStartLSTM(D, H, parallel=parallel).to(dtype)
    if a is not None:
        with torch.no_grad():
            m.a.copy_(torch.as_tensor(a, dtype=dtype))
    return m


def _params(m):
    return [m.weight_ih_l0, m.weight_hh_l0, m.bias_ih_l0, m.bias_hh_l0, m.a]


# ---------------------------------------------------------------------------
def test_init_matches_nn_lstm():
    for D, H in [(16, 24), (64, 128), (7, 5)]:
        torch.manual_seed(3)
        ref = nn.LSTM(D, H)
        torch.manual_seed(3)
        p = O.ref_init_params(D, H, a_init=1e-4)
        for name in ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0"]:
            assert torch.equal(p[name], getattr(ref, name).detach()), name
        assert torch.equal(p["a"], torch.full((4,), 1e-4))
    # RNG consumed by init is exactly the four uniform draws
    torch.manual_seed(5)
    O.ref_init_params(8, 12)
    after = torch.randn(3)
    torch.manual_seed(5)
    nn.LSTM(8, 12)
    assert torch.equal(after, torch.randn(3))


def test_state_dict_layout():
    m = O.RefHeadStartLSTM(16, 24)
    sd = m.state_dict()
    assert list(sd) == ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0", "a"]
    assert [tuple(v.shape) for v in sd.values()] == [(96, 16), (96, 24), (96,), (96,), (4,)]


# ---------------------------------------------------------------------------
def _scalar_cell_T(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a):
    """Plain-Python evaluation of the cell, element by element (tiny sizes)."""
    T, B, D = x.shape
    H = h0.shape[1]
    sig = lambda v: 1.0 / (1.0 + math.exp(-v))
    h = [[float(h0[b, j]) for j in range(H)] for b in range(B)]
    c = [[float(c0[b, j]) for j in range(H)] for b in range(B)]
    outs = []
    for t in range(T):
        nh, nc = [], []
        for b in range(B):
            hb, cb = [], []
            for j in range(H):
                z = []
                for g in range(4):
                    n = g * H + j
                    zi = sum(float(x[t, b, k]) * float(w_ih[n, k]) for k in range(D)) + float(b_ih[n])
                    zr = sum(h[b][k] * float(w_hh[n, k]) for k in range(H)) + float(b_hh[n])
                    z.append(zi + float(a[g]) * zr)
                i, f, gg, o = (sig(v) for v in z)
                cn = f * c[b][j] + i * gg
                hb.append(o * math.tanh(cn))
                cb.append(cn)
            nh.append(hb)
            nc.append(cb)
        h, c = nh, nc
        outs.append(h)
    f64 = torch.float64
    return torch.tensor(outs, dtype=f64), torch.tensor(h, dtype=f64), torch.tensor(c, dtype=f64)


def test_recurrent_forward_scalar_closed_form():
    torch.manual_seed(1)
    D, H, B, T = 3, 4, 2, 2
    m = _model(D, H, a=[0.3, -0.7, 1.1, 0.5])
    x = torch.randn(T, B, D, dtype=torch.float64)
    h0 = torch.randn(B, H, dtype=torch.float64)
    c0 = torch.randn(B, H, dtype=torch.float64)
    out, h_n, c_n = O.recurrent_forward(x, h0, c0, *_params(m))
    e_out, e_h, e_c = _scalar_cell_T(x, h0, c0, *[p.detach() for p in _params(m)])
    assert torch.allclose(out, e_out, atol=1e-12)
    assert torch.allclose(h_n, e_h, atol=1e-12)
    assert torch.allclose(c_n, e_c, atol=1e-12)


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 1e-5)])
def test_recurrent_matches_textbook(dtype, tol):
    """test_cpp.py:55-107: forward and every gradient vs the step-by-step oracle."""
    for (T, B, D, H) in [(10, 4, 16, 24), (8, 3, 8, 12)]:
        m = _model(D, H, dtype=dtype)
        torch.manual_seed(11)
        x = torch.randn(T, B, D, dtype=dtype, requires_grad=True)
        h0 = torch.zeros(B, H, dtype=dtype)
        c0 = torch.zeros(B, H, dtype=dtype)
        out, h_n, c_n = O.recurrent_forward(x, h0, c0, *_params(m))
        (out.sum() + 0.5 * h_n.sum() + 0.25 * c_n.sum()).backward()
        g1 = [p.grad.clone() for p in _params(m)] + [x.grad.clone()]
        for p in _params(m):
            p.grad = None
        x.grad = None
        out2, h2, c2 = O.textbook_forward(x, h0, c0, *_params(m))
        assert (out - out2).abs().max() < tol
        (out2.sum() + 0.5 * h2.sum() + 0.25 * c2.sum()).backward()
        g2 = [p.grad.clone() for p in _params(m)] + [x.grad.clone()]
        for a_, b_ in zip(g1, g2):
            assert (a_ - b_).abs().max() < tol


def test_recurrent_training_step_matches_textbook():
    """test_cpp.py:110-147 in fp64: one SGD step, updated parameters agree."""
    T, B, D, H, lr = 12, 4, 8, 12, 1e-2
    m = _model(D, H)
    ref = [p.detach().clone().requires_grad_(True) for p in _params(m)]
    torch.manual_seed(2)
    x = torch.randn(T, B, D, dtype=torch.float64)
    target = torch.randn(T, B, H, dtype=torch.float64)
    opt = torch.optim.SGD(m.parameters(), lr=lr)
    out, _ = m(x)
    ((out - target) ** 2).mean().backward()
    opt.step()
    out_r, _, _ = O.textbook_forward(x, x.new_zeros(B, H), x.new_zeros(B, H), *ref)
    ((out_r - target) ** 2).mean().backward()
    with torch.no_grad():
        for p in ref:
            p.sub_(lr * p.grad)
    for p, r in zip(_params(m), ref):
        assert (p - r).abs().max() < 1e-10


def test_recurrent_gradcheck():
    torch.manual_seed(4)
    T, B, D, H = 4, 2, 3, 5
    args = [torch.randn(T, B, D, dtype=torch.float64, requires_grad=True),
            torch.randn(B, H, dtype=torch.float64), torch.randn(B, H, dtype=torch.float64)]
    m = _model(D, H, a=[0.4, 0.9, -0.6, 1.3])
    params = [p.detach().clone().requires_grad_(True) for p in _params(m)]
    assert torch.autograd.gradcheck(lambda *a: O.RecurrentRefFn.apply(*a), tuple(args + params),
                                    eps=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
def _rand_gates(B, T, H, seed):
    g = torch.Generator().manual_seed(seed)
    f = torch.rand(B, T, H, generator=g, dtype=torch.float64)
    b = torch.rand(B, T, H, generator=g, dtype=torch.float64)
    c0 = torch.rand(B, 1, H, generator=g, dtype=torch.float64)
    return f, b, c0


@pytest.mark.parametrize("T", [1, 2, 7, 64, 300])
def test_heinsen_scan_is_the_linear_recurrence(T):
    f, b, c0 = _rand_gates(3, T, 5, seed=T)
    c = O.heinsen_scan(f, c0, b)
    lin = O.linear_scan(f.transpose(0, 1), b.transpose(0, 1), c0[:, 0]).transpose(0, 1)
    assert torch.allclose(c, lin, rtol=1e-11, atol=1e-13)


def test_heinsen_scan_product_formula_and_clamps():
    f, b, c0 = _rand_gates(2, 4, 3, seed=9)
    f[0, 1, 0] = 1e-9      # clamped up to eps
    b[1, 2, 2] = 0.0       # clamped up to eps
    c0[0, 0, 1] = -3.0     # clamped up to eps
    c = O.heinsen_scan(f, c0, b)
    eps = O.EPS
    for bb in range(2):
        for j in range(3):
            F = 1.0
            acc = max(float(c0[bb, 0, j]), eps)
            for t in range(4):
                F *= max(float(f[bb, t, j]), eps)
                s = max(float(c0[bb, 0, j]), eps)
                for u in range(t + 1):
                    Fu = 1.0
                    for v in range(u + 1):
                        Fu *= max(float(f[bb, v, j]), eps)
                    s += max(float(b[bb, u, j]), eps) / Fu
                assert math.isclose(float(c[bb, t, j]), F * s, rel_tol=1e-12)
            del acc


def test_parallel_equals_recurrent_at_a0():
    """test_parallel.py:47-60 (+ the exact form: with c0 = eps both compute the same)."""
    T, B, D, H = 12, 3, 16, 24
    m = _model(D, H, a=[0.0] * 4)
    torch.manual_seed(6)
    x = torch.randn(T, B, D, dtype=torch.float64)
    z = x.new_zeros(B, H)
    r = O.recurrent_forward(x, z, z, *_params(m))
    p = O.parallel_forward(x, z, z, *_params(m))
    for u, v in zip(r, p):
        assert (u - v).abs().max() < 1e-4
    c0 = torch.full((B, H), O.EPS, dtype=torch.float64)
    r = O.recurrent_forward(x, z, c0, *_params(m))
    p = O.parallel_forward(x, z, c0, *_params(m))
    for u, v in zip(r, p):
        assert (u - v).abs().max() < 1e-12


def test_parallel_divergence_grows_with_a():
    """test_parallel.py:63-81."""
    T, B, D, H = 12, 3, 16, 24
    torch.manual_seed(7)
    x = torch.randn(T, B, D, dtype=torch.float64)
    z = x.new_zeros(B, H)
    diffs = []
    for a in [0.0, 1e-4, 1e-2, 1e-1, 1.0]:
        m = _model(D, H, a=[a] * 4)
        r, _, _ = O.recurrent_forward(x, z, z, *_params(m))
        p, _, _ = O.parallel_forward(x, z, z, *_params(m))
        diffs.append((r - p).abs().max().item())
    assert diffs[0] < 1e-4
    assert diffs[-1] > 100 * diffs[0]


def test_parallel_backward_matches_recurrent_at_a0():
    """test_parallel.py:84-122: input-path grads agree; W_hh/b_hh/a get none in parallel."""
    T, B, D, H = 10, 3, 8, 12
    m_r = _model(D, H, a=[0.0] * 4)
    m_p = _model(D, H, a=[0.0] * 4, parallel=True)
    torch.manual_seed(8)
    xr = torch.randn(T, B, D, dtype=torch.float64, requires_grad=True)
    xp = xr.detach().clone().requires_grad_(True)
    m_r(xr)[0].sum().backward()
    m_p(xp)[0].sum().backward()
    assert (m_r.weight_ih_l0.grad - m_p.weight_ih_l0.grad).abs().max() < 1e-4
    assert (m_r.bias_ih_l0.grad - m_p.bias_ih_l0.grad).abs().max() < 1e-4
    assert (xr.grad - xp.grad).abs().max() < 1e-4
    assert m_p.weight_hh_l0.grad is None and m_p.bias_hh_l0.grad is None and m_p.a.grad is None


def test_parallel_gradcheck():
    torch.manual_seed(12)
    T, B, D, H = 5, 2, 3, 4
    x = torch.randn(T, B, D, dtype=torch.float64, requires_grad=True)
    c0 = (torch.rand(B, H, dtype=torch.float64) + 0.1).requires_grad_(True)
    m = _model(D, H)
    w_ih = m.weight_ih_l0.detach().clone().requires_grad_(True)
    b_ih = m.bias_ih_l0.detach().clone().requires_grad_(True)
    z = torch.zeros(B, H, dtype=torch.float64)
    fn = lambda x_, c0_, w_, b_: O.parallel_forward(x_, z, c0_, w_, m.weight_hh_l0.detach(), b_,
                                                    m.bias_hh_l0.detach(), m.a.detach())
    assert torch.autograd.gradcheck(fn, (x, c0, w_ih, b_ih), eps=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
@pytest.mark.parametrize("parallel", [False, True])
def test_module_batch_first_and_hx_against_single_rows(parallel):
    """batch_first / hx handling of RefHeadStartLSTM (__init__.py:169-233 of the reference):
    each batch row run alone through the time-major path with a (B,H) = (1,H) state gives
    that row of the batch_first output and of h_n / c_n ((1,B,H))."""
    T, B, D, H = 5, 3, 4, 6
    m = _model(D, H, seed=3, a=0.3 if not parallel else 0.0, parallel=parallel)
    mb = _model(D, H, seed=3, a=0.3 if not parallel else 0.0, parallel=parallel)
    mb.batch_first = True
    g = torch.Generator().manual_seed(7)
    xb = torch.randn(B, T, D, generator=g, dtype=torch.float64)
    h0 = torch.randn(1, B, H, generator=g, dtype=torch.float64) * 0.5
    c0 = torch.rand(1, B, H, generator=g, dtype=torch.float64) + 0.1
    out, (hn, cn) = mb(xb, (h0, c0))
    assert out.shape == (B, T, H) and hn.shape == (1, B, H) and cn.shape == (1, B, H)
    for b in range(B):
        xr = torch.stack([xb[b, t] for t in range(T)]).unsqueeze(1)  # [T, 1, D]
        o1, (h1, c1) = m(xr, (h0[0, b:b + 1], c0[0, b:b + 1]))
        assert torch.allclose(out[b], o1[:, 0], rtol=0, atol=1e-13)
        assert torch.allclose(hn[0, b], h1[0, 0], rtol=0, atol=1e-13)
        assert torch.allclose(cn[0, b], c1[0, 0], rtol=0, atol=1e-13)
    # hx=None is the zero state
    o0, _ = mb(xb)
    oz, _ = mb(xb, (torch.zeros(1, B, H, dtype=torch.float64), torch.zeros(1, B, H, dtype=torch.float64)))
    assert torch.equal(o0, oz)


def test_pins_detect_planted_mistakes(monkeypatch):
    """Each plausible slip in the oracle is caught by one of the pins above."""
    good_bwd = O.cell_backward

    def drop_dc_up(dh, dc_up, c_prev, i, f, g, o, tc):       # forgets the carried dc
        return good_bwd(dh, torch.zeros_like(dc_up), c_prev, i, f, g, o, tc)

    def swap_if(dh, dc_up, c_prev, i, f, g, o, tc):           # i and f grads swapped
        d, dcp = good_bwd(dh, dc_up, c_prev, i, f, g, o, tc)
        H = dh.shape[1]
        return torch.cat([d[:, H:2 * H], d[:, :H], d[:, 2 * H:]], 1), dcp

    torch.manual_seed(4)
    T, B, D, H = 4, 2, 3, 5
    m = _model(D, H, a=[0.4, 0.9, -0.6, 1.3])
    args = (torch.randn(T, B, D, dtype=torch.float64, requires_grad=True),
            torch.randn(B, H, dtype=torch.float64), torch.randn(B, H, dtype=torch.float64),
            *[p.detach().clone().requires_grad_(True) for p in _params(m)])
    for bad in (drop_dc_up, swap_if):
        monkeypatch.setattr(O, "cell_backward", bad)
        assert not torch.autograd.gradcheck(lambda *a: O.RecurrentRefFn.apply(*a), args,
                                            eps=1e-6, atol=1e-7, raise_exception=False)
    monkeypatch.setattr(O, "cell_backward", good_bwd)

    # wrong sign of the cumulative log-f in the scan
    good_scan = O.heinsen_scan

    def bad_scan(f, c0, b, eps=O.EPS):
        return good_scan(1.0 / f.clamp(min=eps), c0, b, eps)
    f, b, c0 = _rand_gates(2, 6, 3, seed=1)
    lin = O.linear_scan(f.transpose(0, 1), b.transpose(0, 1), c0[:, 0]).transpose(0, 1)
    assert not torch.allclose(bad_scan(f, c0, b), lin, rtol=1e-6)
    # a transposed W_hh in the forward
    x = torch.randn(3, 2, 4, dtype=torch.float64)
    mm = _model(4, 4, a=[0.5] * 4)
    p = _params(mm)
    good = O.recurrent_forward(x, x.new_zeros(2, 4), x.new_zeros(2, 4), *p)[0]
    wt = p[1].detach().view(4, 4, 4).transpose(1, 2).reshape(16, 4)
    bad = O.recurrent_forward(x, x.new_zeros(2, 4), x.new_zeros(2, 4), p[0], wt, *p[2:])[0]
    e_out, _, _ = _scalar_cell_T(x, x.new_zeros(2, 4), x.new_zeros(2, 4), *[q.detach() for q in p])
    assert torch.allclose(good, e_out, atol=1e-12) and not torch.allclose(bad, e_out, atol=1e-6)
