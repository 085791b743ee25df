"""Graph-replayed training steps against the CPU oracle.

The benchmark (bench.py) times one replay of a captured forward+backward graph of
the configs[2] module, with x as data (no gradient), so the persistent backward runs
its store_dg=0 branch (weight gradients accumulated inside the kernel, dgates never
written).  These tests run exactly that step and compare every replay with
``oracle.RefHeadStartLSTM`` (the restated reference torch backend, ``_torch.py:86-170``)
on the same inputs, and do the same for the configs[4] parallel step on sampled
channels and for the head-start schedule (``README.md:13-16``, ``__init__.py:156-158``)
with an oracle twin that follows the same SGD updates.
"""

import pytest
import torch

import bench
from conftest import assert_close64, assert_parity, lim_ratio
from oracle import hsl_oracle as O
import prlstm_amd
from prlstm_amd import _lib
from prlstm_amd.graph import GraphedTrainStep

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5
NAMES = ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0", "a"]


def _oracle_step(ref, x):
    """out, h_n, c_n and parameter gradients of loss = out.sum() (the benchmark's loss)."""
    ref.zero_grad(set_to_none=True)
    out, (h_n, c_n) = ref(x)
    out.sum().backward()
    res = {"out": out.detach(), "h_n": h_n.detach(), "c_n": c_n.detach()}
    res.update({"d" + n: p.grad for n, p in ref.named_parameters() if p.grad is not None})
    return res


def test_benched_step_c2_graph_replays_match_oracle(dev):
    """configs[2] built as bench.py builds it, replayed as bench.py replays it, with a fresh
    x per replay; out, h_n, c_n and all five parameter gradients of each replay against the
    fp32 CPU oracle (fp64 tie-break as everywhere)."""
    m_cpu, x0 = bench.make_inputs()
    T, B, D, H = bench.T, bench.B, bench.D, bench.H
    assert tuple(x0.shape) == (T, B, D)
    ref32 = O.RefHeadStartLSTM(D, H, a_init=1e-4)
    ref32.load_state_dict(m_cpu.state_dict())
    ref64 = O.RefHeadStartLSTM(D, H, a_init=1e-4).double()
    ref64.load_state_dict(m_cpu.state_dict())
    m = m_cpu.to(dev)
    step = GraphedTrainStep(m, x0.to(dev))
    g = torch.Generator().manual_seed(11)
    for rep in range(2):
        print(f"c2 graph replay {rep}", flush=True)
        x = torch.randn(T, B, D, generator=g)
        out = step.step(x.to(dev))
        torch.cuda.synchronize()
        got = {"out": out, "h_n": step.static_h_n, "c_n": step.static_c_n}
        got.update({"d" + n: p.grad for n, p in m.named_parameters()})
        assert _lib.last_recurrent_path() == 2
        assert _lib.last_backward_fused() == 2  # dW_hh and dW_ih inside rec_bwd_persistent
        r32 = _oracle_step(ref32, x)
        r64 = _oracle_step(ref64, x.double())
        assert set(r32) == set(got)
        for k in r32:
            assert_parity(f"replay {rep} {k}", got[k].reshape(r32[k].shape), r32[k], r64[k])
    prlstm_amd.check_errors()


def test_benched_step_c4_parallel_graph_replays_match_oracle(dev):
    """configs[4] parallel step (T4096 B16 D256 H1024, a=0) as bench.py's modes table runs it,
    two replays with fresh x: out and c_n on 512 sampled channels, and the rows of dW_ih and
    db_ih of 32 sampled units (all 16 batch rows, 4 gates: 128 of W_ih's 4096 rows), against
    fp64 autograd of the reference formula (_parallel.py:21-74) on the same fp32 inputs.
    dW_ih is a 65536-term sum: as in the other configs[4] tests, the bar is the fp32 CPU
    product of the fp64 dgates with x, or at least as close to fp64 as that product is."""
    T, B, D, H = 4096, 16, 256, 1024
    torch.manual_seed(0)
    m_cpu = prlstm_amd.HeadStartLSTM(D, H, a_init=0.0, parallel=True)
    w_ih = m_cpu.weight_ih_l0.detach().double()
    b_ih = m_cpu.bias_ih_l0.detach().double()
    m = m_cpu.to(dev)
    step = GraphedTrainStep(m, torch.randn(T, B, D).to(dev))
    g = torch.Generator().manual_seed(12)
    units = torch.randperm(H, generator=g)[:32]
    rows = torch.cat([k * H + units for k in range(4)])  # gate-major, as W_ih's rows
    for rep in range(2):
        print(f"c4 parallel graph replay {rep}", flush=True)
        x = torch.randn(T, B, D, generator=g)
        out = step.step(x.to(dev))
        torch.cuda.synchronize()
        # fp64 reference for the sampled units: gates of all batch rows, scan, out.sum()
        w_sub = w_ih[rows].clone().requires_grad_(True)
        b_sub = b_ih[rows].clone().requires_grad_(True)
        gates = (x.double().reshape(T * B, D) @ w_sub.t() + b_sub).view(T, B, 4, len(units))
        gates.retain_grad()
        i, f, gg, o = (torch.sigmoid(gates[:, :, k]) for k in range(4))       # [T, B, n]
        n = B * len(units)
        fl = f.reshape(T, n).t().unsqueeze(-1)
        il = (i * gg).reshape(T, n).t().unsqueeze(-1)
        c = O.heinsen_scan(fl, torch.zeros(n, 1, 1, dtype=torch.float64), il)[..., 0].t().reshape(T, B, -1)
        out_ref = o * torch.tanh(c)
        out_ref.sum().backward()
        got_out = out.cpu()[:, :, units].double()
        got_cn = step.static_c_n.cpu().reshape(B, H)[:, units].double()
        assert_close64("out", got_out, out_ref.detach(), RTOL, ATOL)
        assert_close64("c_n", got_cn, c[-1].detach(), RTOL, ATOL)
        # dW_ih rows: the fp64 product and the fp32 CPU product of the same (fp64) dgates
        dg = gates.grad.reshape(T * B, 4 * len(units))                         # [TB, rows]
        xs = x.reshape(T * B, D)
        want = w_sub.grad
        cpu32 = dg.float().t() @ xs
        got_w = m.weight_ih_l0.grad[rows.to(dev)].cpu()
        print(f"  dW_ih rows: gpu {lim_ratio(got_w, want, RTOL, ATOL):.3g}x, "
              f"cpu fp32 {lim_ratio(cpu32, want, RTOL, ATOL):.3g}x of the tolerance vs fp64", flush=True)
        assert_parity("dW_ih", got_w, cpu32, want, RTOL, ATOL)
        assert_close64("db_ih", m.bias_ih_l0.grad[rows.to(dev)].cpu(), b_sub.grad, RTOL, ATOL)
        for nme in ("weight_hh_l0", "bias_hh_l0", "a"):
            assert getattr(m, nme).grad is None, nme
    prlstm_amd.check_errors()


@pytest.mark.parametrize("shape", [(16, 8, 32, 64), (128, 32, 256, 256)])
def test_head_start_schedule_matches_oracle_twin(dev, shape):
    """The head-start schedule through one GraphedTrainStep (parallel, parallel, recurrent,
    recurrent, parallel, recurrent, SGD after every step) against oracle twins (fp32 and
    fp64 RefHeadStartLSTM) that follow the same schedule with their own gradients: every
    step's output and gradients pass the parity bar, gradients are None exactly where the
    oracle's are, and the parameters after the schedule agree."""
    T, B, D, H = shape
    print(f"schedule vs oracle T={T} B={B} D={D} H={H}", flush=True)
    torch.manual_seed(1)
    ref32 = O.RefHeadStartLSTM(D, H, parallel=True)
    with torch.no_grad():
        ref32.a.fill_(0.2)
    ref64 = O.RefHeadStartLSTM(D, H, parallel=True).double()
    ref64.load_state_dict(ref32.state_dict())
    m = prlstm_amd.HeadStartLSTM(D, H, parallel=True)
    m.load_state_dict(ref32.state_dict())
    m = m.to(dev)
    g = torch.Generator().manual_seed(2)
    xs = [torch.randn(T, B, D, generator=g) for _ in range(6)]
    step = GraphedTrainStep(m, xs[0].to(dev))
    lr = 1e-3
    schedule = [True, True, False, False, True, False]
    for i, (parallel, x) in enumerate(zip(schedule, xs)):
        for mod in (m, ref32, ref64):
            mod.set_mode(parallel)
        out = step.step(x.to(dev))
        torch.cuda.synchronize()
        r32 = _oracle_step(ref32, x)
        r64 = _oracle_step(ref64, x.double())
        got = {"out": out, "h_n": step.static_h_n, "c_n": step.static_c_n}
        got.update({"d" + n: p.grad for n, p in m.named_parameters()})
        for n, p in ref32.named_parameters():
            assert (got["d" + n] is None) == (p.grad is None), (i, n)
        mode = "parallel" if parallel else "recurrent"
        assert set(r32) <= set(got), (set(r32) - set(got))
        for k in r32:
            if parallel:  # fp64 is the bar in parallel mode (the fp32 log-domain scan drifts)
                assert_close64(f"step {i} {mode} {k}", got[k].reshape(r64[k].shape), r64[k], RTOL, ATOL)
            else:
                assert_parity(f"step {i} {mode} {k}", got[k].reshape(r32[k].shape), r32[k], r64[k])
        with torch.no_grad():
            for mod in (m, ref32, ref64):
                for p in mod.parameters():
                    if p.grad is not None:
                        p.add_(p.grad, alpha=-lr)
    for (n, p), q in zip(m.named_parameters(), ref64.parameters()):
        assert lim_ratio(p.detach().cpu(), q.detach(), 1e-6, 1e-7) <= 1.0, n
    assert set(step._graphs) == {True, False}
    prlstm_amd.check_errors()
