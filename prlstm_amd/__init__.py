"""HeadStartLSTM on MI355X (gfx950): the training hot path as hand-written HIP kernels.

HeadStartLSTM is a single-layer, unidirectional LSTM with two changes from
``torch.nn.LSTM``: the g-gate uses sigmoid, and the recurrent term
``W_hh h_{t-1} + b_hh`` is scaled by a learnable per-gate ``a = [a_i, a_f, a_g, a_o]``.
With ``parallel=True`` the a-term is dropped and the cell state becomes a
positive first-order linear recurrence, solved as a scan over time.

This package keeps the reference module's API (``src/headstartlstm/__init__.py:99-233``):
the constructor arguments, the ``nn.LSTM``-compatible parameters
``weight_ih_l0, weight_hh_l0, bias_ih_l0, bias_hh_l0`` plus ``a`` (same order,
same init and RNG use), ``set_mode(parallel=...)`` and
``forward(x, hx=None) -> (output, (h_n, c_n))``.  Every forward and backward runs
on the HIP kernels of ``libhsl.so``; CPU tensors are rejected.
"""

import math

import torch
import torch.nn as nn

from .functional import EPS, headstartlstm_parallel, headstartlstm_recurrent
from ._lib import (check_errors, last_recurrent_path, set_exchange_scope, set_recurrent_path, set_spin_timeout_us,
                   set_split_products)

__version__ = "0.1.0"


class HeadStartLSTM(nn.Module):
    """An LSTM with a parallel-scan mode that warm-starts BPTT training.

    Parameters (as the reference, ``__init__.py:104-127``)
    ----------
    input_size, hidden_size : int
    batch_first : bool, default False -- input is [B, T, D] instead of [T, B, D]
    a_init : float, default 1e-4 -- initial value of the per-gate scale ``a``
    backend : {"auto", "torch", "cpp", "triton", "metal"}, default "auto"
        Accepted for signature compatibility and validated like the reference;
        every value runs the MI355X HIP kernels.
    parallel : bool, default False -- start in parallel-scan mode
    compile_cell : bool, default False -- accepted and ignored (the cell is
        already one fused kernel)
    """

    _VALID_BACKENDS = ("auto", "torch", "cpp", "triton", "metal")

    def __init__(self, input_size, hidden_size, batch_first=False, a_init=1e-4,
                 backend="auto", parallel=False, compile_cell=False):
        super().__init__()
        assert backend in self._VALID_BACKENDS, (
            f"backend must be one of {self._VALID_BACKENDS}, got {backend!r}")
        self.input_size = input_size
        self.hidden_size = hidden_size
        self.batch_first = batch_first
        self.a_init = a_init
        self.backend = backend
        self.parallel = parallel
        self.compile_cell = compile_cell
        H, D = hidden_size, input_size
        # nn.LSTM names and layout, gate order [i, f, g, o] (__init__.py:147-152)
        self.weight_ih_l0 = nn.Parameter(torch.empty(4 * H, D))
        self.weight_hh_l0 = nn.Parameter(torch.empty(4 * H, H))
        self.bias_ih_l0 = nn.Parameter(torch.zeros(4 * H))
        self.bias_hh_l0 = nn.Parameter(torch.zeros(4 * H))
        self.a = nn.Parameter(torch.full((4,), float(a_init)))
        self.reset_parameters()

    def set_mode(self, parallel: bool):
        """Switch between recurrent (default) and parallel-scan mode."""
        self.parallel = parallel

    def reset_parameters(self):
        """nn.LSTM init U(-1/sqrt(H), 1/sqrt(H)) on the weights and biases, a = a_init."""
        bound = 1.0 / math.sqrt(self.hidden_size)
        for p in (self.weight_ih_l0, self.weight_hh_l0, self.bias_ih_l0, self.bias_hh_l0):
            nn.init.uniform_(p, -bound, bound)
        with torch.no_grad():
            self.a.fill_(self.a_init)

    def forward(self, x, hx=None):
        if self.batch_first:
            x = x.transpose(0, 1).contiguous()
        T, B, _ = x.shape
        if hx is None:
            h0 = c0 = None  # zero initial states, passed to the kernels as NULL
        else:
            h0, c0 = hx
            if h0.dim() == 3:
                h0 = h0.squeeze(0)
            if c0.dim() == 3:
                c0 = c0.squeeze(0)
        fn = headstartlstm_parallel if self.parallel else headstartlstm_recurrent
        output, h_n, c_n = fn(x, h0, c0, self.weight_ih_l0, self.weight_hh_l0,
                              self.bias_ih_l0, self.bias_hh_l0, self.a)
        if self.batch_first:
            output = output.transpose(0, 1).contiguous()
        return output, (h_n.unsqueeze(0), c_n.unsqueeze(0))

    def extra_repr(self):
        return (f"{self.input_size}, {self.hidden_size}, batch_first={self.batch_first}, "
                f"parallel={self.parallel}")


__all__ = [
    "HeadStartLSTM", "headstartlstm_recurrent", "headstartlstm_parallel", "EPS",
    "set_recurrent_path", "set_spin_timeout_us", "set_exchange_scope", "set_split_products", "last_recurrent_path",
    "check_errors",
    "__version__",
]
