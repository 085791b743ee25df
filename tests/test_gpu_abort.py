"""A persistent kernel that gives up a wait fails loudly.

The persistent recurrent kernels bound every wait for another workgroup
(``hsl_set_spin_timeout_us``).  When one gives up, the reference would have failed
loudly (``TORCH_CHECK`` at ``_csrc/lstm_cell.cpp:38-43``, ``RuntimeError`` at
``_metal.py:85-87``); here the aborting workgroups fill every output they own with NaN
and raise the sticky device word that ``prlstm_amd.check_errors`` reads, so the loss
and the gradients of that call are NaN, never silently wrong.

The condition is forced from the host with a 1 us spin limit: the workgroups then give
up their first waits (the kernel start alone spreads their arrival by more than that)
and every kernel exits normally.  After the limit is restored, the same module must
run cleanly again.
"""

import pytest
import torch

import prlstm_amd
from prlstm_amd import _lib
from prlstm_amd.graph import GraphedTrainStep

pytestmark = pytest.mark.gpu


@pytest.fixture
def tiny_spin():
    prlstm_amd.check_errors()  # nothing pending from earlier tests
    prev = prlstm_amd.set_spin_timeout_us(1)
    yield
    prlstm_amd.set_spin_timeout_us(prev)
    _lib.device_errors(clear=True)


def _finite(t):
    return t is None or bool(torch.isfinite(t).all())


def _step(m, x):
    m.zero_grad(set_to_none=True)
    out, (h_n, c_n) = m(x)
    out.sum().backward()
    torch.cuda.synchronize()
    return out.detach(), [p.grad for p in m.parameters()]


def test_timed_out_waits_poison_outputs_and_raise(dev, tiny_spin):
    T, B, D, H = 64, 32, 256, 512
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(D, H).to(dev)
    x = torch.randn(T, B, D, device=dev)
    aborted = 0
    for attempt in range(3):
        print(f"abort attempt {attempt}", flush=True)
        out, grads = _step(m, x)
        assert _lib.last_recurrent_path() == 2
        flags = _lib.device_errors(clear=False)
        all_finite = _finite(out) and all(_finite(g) for g in grads)
        if flags:
            assert flags & 1
            assert not all_finite, "a call whose waits gave up returned finite results"
            with pytest.raises(RuntimeError, match="gave up a wait"):
                prlstm_amd.check_errors()
            aborted += 1
        else:
            assert all_finite
    assert aborted >= 1, "a 1 us spin limit never made a persistent wait give up"
    # restored limit: a clean, finite step and no error
    prlstm_amd.set_spin_timeout_us(2_000_000)
    out, grads = _step(m, x)
    prlstm_amd.check_errors()
    assert _finite(out) and all(_finite(g) for g in grads)


def test_timed_out_waits_in_graph_replay(dev, tiny_spin):
    """A graph captured while the limit is 1 us keeps it in its kernel arguments: a replay
    whose waits give up returns NaN and raises the device word (and one that does not
    returns finite results); a graph captured after the limit is restored replays
    cleanly."""
    T, B, D, H = 64, 32, 256, 512
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(D, H).to(dev)
    x = torch.randn(T, B, D, device=dev)
    step = GraphedTrainStep(m, x)
    _lib.device_errors(clear=True)  # the eager warm-up steps of the capture ran with 1 us too
    bad = 0
    for rep in range(3):
        out = step.step(x)
        torch.cuda.synchronize()
        flags = _lib.device_errors(clear=True)
        finite = _finite(out) and all(_finite(p.grad) for p in m.parameters())
        assert bool(flags) != finite, (rep, flags, finite)
        bad += bool(flags)
    assert bad >= 1
    prlstm_amd.set_spin_timeout_us(2_000_000)
    step = GraphedTrainStep(m, x)
    out = step.step(x)
    torch.cuda.synchronize()
    prlstm_amd.check_errors()
    assert _finite(out) and all(_finite(p.grad) for p in m.parameters())


@pytest.mark.parametrize("H,B", [(2048, 8), (2048, 24), (1024, 24)])
def test_timed_out_waits_wide_kernels(dev, tiny_spin, H, B):
    """The W_hh-resident kernels (rec_fwd_wide, and rec_bwd_wide at H = 2048 or rec_bwd_wide1
    at H = 1024) bound their waits the same way: an aborting workgroup fills what it owns
    with NaN and raises the device word.  B = 8 runs one batch chain, B = 24 two.  The
    forward is checked alone, then forward + backward.  32 steps: the two-chain kernels hide
    most hand-offs, so a short launch may finish every wait within the 1 us limit."""
    T, D = 32, 32
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(D, H).to(dev)
    x = torch.randn(T, B, D, device=dev)
    aborted = 0
    for attempt in range(5):
        print(f"wide forward abort attempt {attempt}", flush=True)
        with torch.no_grad():
            out, (h_n, c_n) = m(x)
        torch.cuda.synchronize()
        assert _lib.last_recurrent_path() == 3
        flags = _lib.device_errors(clear=True)
        finite = _finite(out) and _finite(h_n) and _finite(c_n)
        assert bool(flags) != finite, (attempt, flags, finite)
        aborted += bool(flags)
    assert aborted >= 1, "a 1 us spin limit never made the wide forward give up a wait"
    aborted = 0
    for attempt in range(5):
        print(f"wide step abort attempt {attempt}", flush=True)
        out, grads = _step(m, x)
        assert _lib.last_recurrent_path() == 3
        flags = _lib.device_errors(clear=True)
        finite = _finite(out) and all(_finite(g) for g in grads)
        assert bool(flags) != finite, (attempt, flags, finite)
        aborted += bool(flags)
    assert aborted >= 1, "a 1 us spin limit never made the wide kernels give up a wait"
    prlstm_amd.set_spin_timeout_us(2_000_000)
    out, grads = _step(m, x)
    prlstm_amd.check_errors()
    assert _finite(out) and all(_finite(g) for g in grads)
