"""Whole-step graph capture: forward + backward of a HeadStartLSTM in one HIP graph.

The reference captures the forward and backward time loops as two CUDA graphs
with static buffers that are cloned out on every call (``_triton.py:205-321``,
``:365-378``).  Here the time loops are already single persistent launches, so
the graph holds the entire training step -- input projection, recurrence or
scan, BPTT, weight-gradient GEMMs and reductions -- and replays it with one
host call.

The head-start schedule trains in parallel mode first and then switches to
recurrent mode with ``set_mode`` (``__init__.py:156-158``).  The step keeps one
graph per mode, captured the first time that mode is stepped (the cache key is
the module's ``parallel`` flag), each with its own static buffers, including the
gradient tensors autograd allocates during its capture.  After every replay the
parameters' ``.grad`` point at the gradients of the mode just replayed, or are
``None`` for parameters that mode does not use (``W_hh``, ``b_hh`` and ``a`` in
parallel mode), exactly as an eager step leaves them.
"""

import torch


class GraphedTrainStep:
    """Capture ``loss = sum(grad_out * module(x)[0])`` forward+backward for fixed shapes.

    ``grad_out`` defaults to ones, i.e. the gradient of ``output.sum()``
    (the loss the reference's tests and benchmarks use).  The loss value itself
    is not computed inside the graph: only its gradient is needed for the
    parameter update, and keeping reductions out of the graph avoids library
    kernels that record memset nodes.

    The caller passes new inputs to ``step`` (or copies them into ``static_x``)
    and updates the parameters in place between steps, as optimizers do.
    """

    def __init__(self, module, example_x, hx=None, grad_out=None, warmup=2):
        self.module = module
        self.static_x = example_x.detach().clone()
        self.hx = hx
        self.warmup = warmup
        with torch.no_grad():
            out, _ = module(self.static_x, hx)
        self.grad_out = torch.ones_like(out) if grad_out is None else grad_out.detach().clone()
        self._graphs = {}
        self.static_out = self.static_h_n = self.static_c_n = None
        self._capture(bool(module.parallel))

    def _capture(self, mode):
        m = self.module
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(self.warmup):
                m.zero_grad(set_to_none=True)
                out, hc = m(self.static_x, self.hx)
                torch.autograd.backward([out], [self.grad_out])
                del out, hc
        torch.cuda.current_stream().wait_stream(side)
        m.zero_grad(set_to_none=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out, (h_n, c_n) = m(self.static_x, self.hx)
            torch.autograd.backward([out], [self.grad_out])
        grads = {n: p.grad for n, p in m.named_parameters()}
        # Only detached views of the static outputs are kept (same memory): the captured
        # autograd graph, and with it the parameters' AccumulateGrad nodes created on the
        # capture stream, is released, so later eager steps on another stream build their
        # own nodes instead of reusing those (a stream mismatch torch warns about).
        self._graphs[mode] = (graph, out.detach(), h_n.detach(), c_n.detach(), grads)
        del out, h_n, c_n

    @property
    def graph(self):
        """The graph of the module's current mode (captured on first use)."""
        mode = bool(self.module.parallel)
        if mode not in self._graphs:
            self._capture(mode)
        return self._graphs[mode][0]

    def step(self, x=None):
        """Replay the step of the module's current mode; returns its (static) output tensor."""
        mode = bool(self.module.parallel)
        if mode not in self._graphs:
            self._capture(mode)
        graph, out, h_n, c_n, grads = self._graphs[mode]
        if x is not None:
            self.static_x.copy_(x)
        graph.replay()
        for n, p in self.module.named_parameters():
            p.grad = grads[n]
        self.static_out, self.static_h_n, self.static_c_n = out, h_n, c_n
        return out
