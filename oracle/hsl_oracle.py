"""CPU oracle for the HeadStartLSTM training hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``prlstm_amd``) may import,
call or link this module.  It is used by ``tests/`` (as the checker),
``__graft_entry__.smoke()`` (as the checker) and ``bench.py`` (the timed
``cpu_baseline`` leg).  It is never the thing measured on the GPU and never a
fallback for the GPU path.

It restates, with torch CPU ops in the same operation order (so that the fp32
rounding matches the reference's CPU run on the same torch build), the
reference ``torch`` backend and the parallel-scan mode of HeadStartLSTM:

* ``ref_init_params``        -- ``__init__.py:147-167`` (parameter order, nn.LSTM
                                 uniform init, RNG consumption, ``a`` fill)
* ``RecurrentRefFn``         -- ``_torch.py:86-170`` (a-prescale, one input GEMM,
                                 T-step loop, hand-written BPTT, batched grads)
* ``cell_forward`` /
  ``cell_backward``          -- ``_torch.py:27-53``
* ``heinsen_scan``           -- ``_parallel.py:21-35``
* ``parallel_forward``       -- ``_parallel.py:38-74`` (autograd-traced backward)
* ``RefHeadStartLSTM``       -- ``__init__.py:131-233`` (hx / batch_first handling)
* ``textbook_forward``       -- ``tests/test_cpp.py:25-48`` (the reference's own
                                 step-by-step oracle; independent of the above)
* ``linear_scan``            -- the first-order linear recurrence that the
                                 Heinsen formula evaluates in closed form
                                 (``_parallel.py:9-16``), used to pin it.

Each function runs in fp32 or fp64 (whatever dtype its inputs carry).  How each
one is pinned (known answers, invariants, fp64 gradcheck, brute force) is
recorded in ``tests/test_oracle.py``.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

EPS = 1e-6  # clamp floor of the log-domain scan (_parallel.py:21, :38)


# ---------------------------------------------------------------------------
# parameters (__init__.py:147-167)
# ---------------------------------------------------------------------------
def ref_init_params(input_size, hidden_size, a_init=1e-4):
    """Create the five parameters the way the reference module does.

    Order of creation and of the uniform draws: weight_ih_l0, weight_hh_l0,
    bias_ih_l0, bias_hh_l0 (U(-1/sqrt(H), 1/sqrt(H)) each), then ``a`` is
    filled with ``a_init`` (``__init__.py:148-152``, ``:160-167``).
    """
    H, D = hidden_size, input_size
    w_ih = torch.empty(4 * H, D)
    w_hh = torch.empty(4 * H, H)
    b_ih = torch.zeros(4 * H)
    b_hh = torch.zeros(4 * H)
    a = torch.full((4,), float(a_init))
    bound = 1.0 / math.sqrt(H)
    for p in (w_ih, w_hh, b_ih, b_hh):
        nn.init.uniform_(p, -bound, bound)
    a.fill_(a_init)
    return {"weight_ih_l0": w_ih, "weight_hh_l0": w_hh,
            "bias_ih_l0": b_ih, "bias_hh_l0": b_hh, "a": a}


# ---------------------------------------------------------------------------
# recurrent mode (_torch.py)
# ---------------------------------------------------------------------------
def cell_forward(gates, c_prev):
    """One cell step (_torch.py:27-36): sigmoid on all four gates, g included."""
    gi, gf, gg, go = gates.chunk(4, dim=1)
    i = torch.sigmoid(gi)
    f = torch.sigmoid(gf)
    g = torch.sigmoid(gg)
    o = torch.sigmoid(go)
    c = f * c_prev + i * g
    tc = torch.tanh(c)
    h = o * tc
    return h, c, i, f, g, o, tc


def cell_backward(dh, dc_up, c_prev, i, f, g, o, tc):
    """Cell backward (_torch.py:39-53); returns (dgates [B,4H], dc_prev)."""
    d_o = dh * tc
    dc = dc_up + dh * o * (1.0 - tc * tc)
    d_f = dc * c_prev
    dc_prev = dc * f
    d_i = dc * g
    d_g = dc * i
    pre_i = d_i * i * (1.0 - i)
    pre_f = d_f * f * (1.0 - f)
    pre_g = d_g * g * (1.0 - g)
    pre_o = d_o * o * (1.0 - o)
    return torch.cat([pre_i, pre_f, pre_g, pre_o], dim=1), dc_prev


class RecurrentRefFn(torch.autograd.Function):
    """Restatement of HeadStartLSTMTorchFn (_torch.py:86-170).

    Backward returns None for h0 and c0, as the reference does (_torch.py:170).
    """

    @staticmethod
    def forward(ctx, x, h0, c0, w_ih, w_hh, b_ih, b_hh, a):
        T, B, _ = x.shape
        H = h0.shape[-1]
        a_rep = a.repeat_interleave(H)
        w_hh_s = a_rep.unsqueeze(1) * w_hh
        b_hh_s = a_rep * b_hh
        w_hh_s_t = w_hh_s.t().contiguous()
        gih = F.linear(x, w_ih, b_ih)
        hs = x.new_zeros(T + 1, B, H)
        cs = x.new_zeros(T + 1, B, H)
        acts = [x.new_zeros(T, B, H) for _ in range(5)]   # i, f, g, o, tanh_c
        hs[0].copy_(h0)
        cs[0].copy_(c0)
        h, c = h0, c0
        for t in range(T):
            gates = gih[t] + h @ w_hh_s_t + b_hh_s
            h, c, *step_acts = cell_forward(gates, c)
            hs[t + 1] = h
            cs[t + 1] = c
            for buf, v in zip(acts, step_acts):
                buf[t] = v
        ctx.save_for_backward(x, hs, cs, *acts, w_ih, w_hh, b_ih, b_hh, a, w_hh_s, a_rep)
        return hs[1:], hs[T], cs[T]

    @staticmethod
    def backward(ctx, dout, dh_n, dc_n):
        (x, hs, cs, i_s, f_s, g_s, o_s, tc_s,
         w_ih, w_hh, b_ih, b_hh, a, w_hh_s, a_rep) = ctx.saved_tensors
        T, B, D = x.shape
        H = hs.shape[-1]
        dg_all = x.new_zeros(T, B, 4 * H)
        dh = dh_n.contiguous().clone()
        dc = dc_n.contiguous().clone()
        for t in range(T - 1, -1, -1):
            dh = dh + dout[t]
            dg, dc = cell_backward(dh, dc, cs[t], i_s[t], f_s[t], g_s[t], o_s[t], tc_s[t])
            dg_all[t] = dg
            dh = dg @ w_hh_s
        dg2 = dg_all.view(T * B, 4 * H)
        hp2 = hs[:-1].reshape(T * B, H)
        x2 = x.view(T * B, D)
        dw_hh_s = dg2.t() @ hp2
        dw_ih = dg2.t() @ x2
        db = dg2.sum(dim=0)
        dx = (dg2 @ w_ih).view(T, B, D)
        dw_hh = a_rep.unsqueeze(1) * dw_hh_s
        db_hh = a_rep * db
        da = ((w_hh * dw_hh_s).sum(dim=1) + b_hh * db).view(4, H).sum(dim=1)
        return dx, None, None, dw_ih, dw_hh, db, db_hh, da


def recurrent_forward(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a):
    """Functional form of the reference torch backend (_torch.py:173-176)."""
    return RecurrentRefFn.apply(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a)


# ---------------------------------------------------------------------------
# parallel mode (_parallel.py)
# ---------------------------------------------------------------------------
def heinsen_scan(f, c0, b, eps=EPS):
    """Log-domain prefix scan of c_t = f_t c_{t-1} + b_t (_parallel.py:21-35).

    f, b: [B, T, H]; c0: [B, 1, H].  Returns c [B, T, H].
    """
    lf = torch.log(torch.clamp(f, min=eps))
    lb = torch.log(torch.clamp(b, min=eps))
    lc0 = torch.log(torch.clamp(c0, min=eps))
    astar = torch.cumsum(lf, dim=1)
    seq = torch.cat([lc0, lb - astar], dim=1)
    tail = torch.logcumsumexp(seq, dim=1)[:, 1:]
    return torch.exp(astar + tail)


def parallel_forward(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a, eps=EPS):
    """Parallel-mode forward (_parallel.py:38-74).  h0, w_hh, b_hh, a unused."""
    gates = F.linear(x, w_ih, b_ih)
    gi, gf, gg, go = gates.chunk(4, dim=-1)
    i = torch.sigmoid(gi)
    f = torch.sigmoid(gf)
    g = torch.sigmoid(gg)
    o = torch.sigmoid(go)
    b = i * g
    c_bth = heinsen_scan(f.transpose(0, 1).contiguous(), c0.unsqueeze(1),
                         b.transpose(0, 1).contiguous(), eps=eps)
    c = c_bth.transpose(0, 1).contiguous()
    out = o * torch.tanh(c)
    return out, out[-1].contiguous(), c[-1].contiguous()


def linear_scan(f, b, c0, eps=EPS):
    """c_t = max(f_t,eps) c_{t-1} + max(b_t,eps), c_{-1} = max(c0,eps), along dim 0.

    f, b: [T, ...]; c0: [...].  This is the recurrence whose closed form the
    Heinsen scan evaluates (_parallel.py:9-16); it pins ``heinsen_scan``.
    """
    c = torch.clamp(c0, min=eps)
    fc = torch.clamp(f, min=eps)
    bc = torch.clamp(b, min=eps)
    out = []
    for ft, bt in zip(fc.unbind(0), bc.unbind(0)):  # unbind: one stacked gradient in backward
        c = ft * c + bt
        out.append(c)
    return torch.stack(out, 0)


# ---------------------------------------------------------------------------
# the reference's own step-by-step oracle (tests/test_cpp.py:25-48)
# ---------------------------------------------------------------------------
def textbook_forward(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a):
    """Per-step F.linear cell, differentiated by autograd (test_cpp.py:25-48)."""
    T = x.shape[0]
    H = h0.shape[-1]
    a_rep = a.repeat_interleave(H)
    w_hh_s = a_rep.unsqueeze(1) * w_hh
    b_hh_s = a_rep * b_hh
    h, c = h0, c0
    outs = []
    for t in range(T):
        z = F.linear(x[t], w_ih, b_ih) + F.linear(h, w_hh_s, b_hh_s)
        zi, zf, zg, zo = z.chunk(4, dim=1)
        c = torch.sigmoid(zf) * c + torch.sigmoid(zi) * torch.sigmoid(zg)
        h = torch.sigmoid(zo) * torch.tanh(c)
        outs.append(h)
    return torch.stack(outs, 0), h, c


# ---------------------------------------------------------------------------
# module (__init__.py:99-233), CPU only
# ---------------------------------------------------------------------------
class RefHeadStartLSTM(nn.Module):
    """CPU restatement of the reference module, used as the checker and the
    timed CPU baseline.  Same parameter names, order, init and forward
    semantics (batch_first transpose, hx squeeze, (h_n, c_n) unsqueeze)."""

    def __init__(self, input_size, hidden_size, batch_first=False, a_init=1e-4,
                 parallel=False):
        super().__init__()
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.batch_first = batch_first
        self.a_init = a_init
        self.parallel = parallel
        p = ref_init_params(input_size, hidden_size, a_init)
        for name, v in p.items():
            setattr(self, name, nn.Parameter(v))

    def set_mode(self, parallel):
        self.parallel = parallel

    def forward(self, x, hx=None):
        if self.batch_first:
            x = x.transpose(0, 1).contiguous()
        T, B, _ = x.shape
        if hx is None:
            h0 = x.new_zeros(B, self.hidden_size)
            c0 = x.new_zeros(B, self.hidden_size)
        else:
            h0, c0 = hx
            if h0.dim() == 3:
                h0 = h0.squeeze(0)
            if c0.dim() == 3:
                c0 = c0.squeeze(0)
        fn = parallel_forward if self.parallel else recurrent_forward
        out, h_n, c_n = fn(x, h0, c0, self.weight_ih_l0, self.weight_hh_l0,
                           self.bias_ih_l0, self.bias_hh_l0, self.a)
        if self.batch_first:
            out = out.transpose(0, 1).contiguous()
        return out, (h_n.unsqueeze(0), c_n.unsqueeze(0))
