"""Whole-step graph capture: forward + backward of a HeadStartLSTM in one HIP graph.

The reference captures the forward and backward time loops as two CUDA graphs
with static buffers that are cloned out on every call (``_triton.py:205-321``,
``:365-378``).  Here the time loops are already single persistent launches, so
the graph holds the entire training step -- input projection, recurrence or
scan, BPTT, weight-gradient GEMMs and reductions -- and replays it with one
host call.  The caller copies new inputs into ``static_x`` (or passes them to
``step``); gradients land in the parameters' ``.grad`` tensors, which the graph
owns after capture.
"""

import torch


class GraphedTrainStep:
    """Capture ``loss = sum(grad_out * module(x)[0])`` forward+backward for fixed shapes.

    ``grad_out`` defaults to ones, i.e. the gradient of ``output.sum()``
    (the loss the reference's tests and benchmarks use).  The loss value itself
    is not computed inside the graph: only its gradient is needed for the
    parameter update, and keeping reductions out of the graph avoids library
    kernels that record memset nodes.
    """

    def __init__(self, module, example_x, hx=None, grad_out=None, warmup=2):
        self.module = module
        self.static_x = example_x.detach().clone()
        self.hx = hx
        with torch.no_grad():
            out, _ = module(self.static_x, hx)
        self.grad_out = torch.ones_like(out) if grad_out is None else grad_out.detach().clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                module.zero_grad(set_to_none=True)
                out, hc = module(self.static_x, hx)
                torch.autograd.backward([out], [self.grad_out])
                del out, hc
        torch.cuda.current_stream().wait_stream(side)
        module.zero_grad(set_to_none=True)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            out, (h_n, c_n) = module(self.static_x, hx)
            torch.autograd.backward([out], [self.grad_out])
        self.static_out = out
        self.static_h_n = h_n
        self.static_c_n = c_n

    def step(self, x=None):
        """Replay the captured step; returns the (static) output tensor."""
        if x is not None:
            self.static_x.copy_(x)
        self.graph.replay()
        return self.static_out
