"""Autograd functions of the HeadStartLSTM hot path on MI355X.

Both keep the reference backend functional signature
``fn(x, h0, c0, W_ih, W_hh, b_ih, b_hh, a) -> (output[T,B,H], h_n[B,H], c_n[B,H])``
(``_torch.py:173``, ``_parallel.py:38``) and run every kernel through libhsl
(include/hsl.h) on the current HIP stream.  No host synchronisation and no
allocation outside torch's caching allocator happens, so a whole training step
can be captured in a graph (see ``prlstm_amd.graph``).
"""

import ctypes

import torch

from . import _lib

EPS = 1e-6  # clamp floor of the parallel scan (_parallel.py:21, :38)

_debug_checks = False


def debug_checks(enabled=True):
    """When enabled, every recurrent call synchronises and raises if a persistent
    kernel reported a timed-out wait (the device error flag of its workspace, and the
    sticky device word that ``prlstm_amd.check_errors`` reads).  Without it a timed-out
    call is still not silent: its outputs are NaN."""
    global _debug_checks
    _debug_checks = bool(enabled)


def _poll(ws, device):
    if not _debug_checks:
        return
    flag = ctypes.c_int(0)
    _lib.call("hsl_poll_error", _lib.ptr(ws), ctypes.byref(flag), _lib.stream_of(device))
    if flag.value:
        _lib.device_errors(device, clear=True)
        raise RuntimeError(f"a persistent kernel reported device error flag {flag.value} "
                           "(a wait between workgroups timed out); its outputs are NaN")


def _check(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a):
    if x.dim() != 3:
        raise RuntimeError(f"x must be [T, B, D], got shape {tuple(x.shape)}")
    T, B, D = x.shape
    H = w_hh.shape[-1]
    want = {
        "h0": (h0, (B, H)), "c0": (c0, (B, H)),
        "weight_ih_l0": (w_ih, (4 * H, D)), "weight_hh_l0": (w_hh, (4 * H, H)),
        "bias_ih_l0": (b_ih, (4 * H,)), "bias_hh_l0": (b_hh, (4 * H,)), "a": (a, (4,)),
    }
    want = {k: v for k, v in want.items() if v[0] is not None}  # h0/c0 None: zero states
    for name, (t, shape) in want.items():
        if tuple(t.shape) != shape:
            raise RuntimeError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    for name, t in [("x", x)] + [(n, v[0]) for n, v in want.items()]:
        if t.device.type != "cuda":
            raise RuntimeError(
                f"prlstm_amd runs on ROCm devices only: {name} is on {t.device} "
                "(move the module and inputs to the GPU)")
        if t.device != x.device:
            raise RuntimeError(f"{name} is on {t.device}, x is on {x.device}")
        if t.dtype != x.dtype or x.dtype not in (torch.float32, torch.float64):
            raise RuntimeError(f"prlstm_amd kernels compute in float32 or float64 (bf16/fp16 modules are "
                               f"widened at the functional), every operand in x's dtype; {name} is {t.dtype}, "
                               f"x is {x.dtype}")
    return T, B, D, H


def _entry(name, x):
    """The C-ABI entry point for x's dtype: name, or its fp64 twin name + '_f64'."""
    return name + "_f64" if x.dtype == torch.float64 else name


def _c(t):
    return t if t is None or t.is_contiguous() else t.contiguous()


def _grad_or_zeros(g, like):
    return _c(g) if g is not None else torch.zeros_like(like)

# h0/c0 may be None (zero initial states) and the gradients of h_n/c_n arrive as None
# when the loss does not use them (set_materialize_grads(False)); both reach the C ABI
# as NULL, which it reads as zeros, so no zero tensors are filled per step.


class RecurrentFn(torch.autograd.Function):
    """Exact BPTT (the reference torch backend, ``_torch.py:86-170``).

    Backward returns gradients for x, the four weights/biases and a, plus the
    gradients w.r.t. h0 and c0 when those require grad (the reference torch
    backend returns None for them; its Metal backend returns them).
    """

    @staticmethod
    def forward(ctx, x, h0, c0, w_ih, w_hh, b_ih, b_hh, a):
        T, B, D, H = _check(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a)
        x, h0, c0, w_ih, w_hh, b_ih, b_hh, a = map(_c, (x, h0, c0, w_ih, w_hh, b_ih, b_hh, a))
        if x.data_ptr() % 16:  # the workspace query assumes a 16-byte aligned x
            x = x.clone()
        ctx.set_materialize_grads(False)
        h_save = x.new_empty(T + 1, B, H)
        c_save = x.new_empty(T + 1, B, H)
        gact = x.new_empty(T, B, H, 4)
        tanh_c = x.new_empty(T, B, H)
        lib = _lib.load()
        f64 = x.dtype == torch.float64
        nbytes = (lib.hsl_rec_fwd_f64_ws_bytes if f64 else lib.hsl_rec_fwd_ws_bytes)(T, B, D, H)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        P = _lib.ptr
        _lib.call(_entry("hsl_rec_fwd", x), P(x), P(h0), P(c0), P(w_ih), P(w_hh), P(b_ih), P(b_hh), P(a),
                  P(h_save), P(c_save), P(gact), P(tanh_c), P(ws), nbytes, T, B, D, H,
                  _lib.stream_of(x.device))
        if not f64:  # the fp64 kernels have no waits between workgroups
            _poll(ws, x.device)
        ctx.save_for_backward(x, w_ih, w_hh, b_hh, a, h_save, c_save, gact, tanh_c)
        ctx.dims = (T, B, D, H)
        return h_save[1:], h_save[T], c_save[T]

    @staticmethod
    def backward(ctx, dout, dh_n, dc_n):
        x, w_ih, w_hh, b_hh, a, h_save, c_save, gact, tanh_c = ctx.saved_tensors
        T, B, D, H = ctx.dims
        dout = _grad_or_zeros(dout, h_save[1:])
        dh_n, dc_n = _c(dh_n), _c(dc_n)
        need = ctx.needs_input_grad
        dx = torch.empty_like(x) if need[0] else None
        dh0 = x.new_empty(B, H) if need[1] else None
        dc0 = x.new_empty(B, H) if need[2] else None
        dw_ih = torch.empty_like(w_ih)
        dw_hh = torch.empty_like(w_hh)
        db_ih = x.new_empty(4 * H)
        db_hh = x.new_empty(4 * H)
        da = x.new_empty(4)
        lib = _lib.load()
        f64 = x.dtype == torch.float64
        nbytes = (lib.hsl_rec_bwd_f64_ws_bytes(T, B, D, H) if f64
                  else lib.hsl_rec_bwd_ws_bytes_for(T, B, D, H, 1 if dx is not None else 0))
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        P = _lib.ptr
        _lib.call(_entry("hsl_rec_bwd", x), P(dout), P(dh_n), P(dc_n), P(x), P(h_save), P(c_save), P(gact),
                  P(tanh_c), P(w_ih), P(w_hh), P(b_hh), P(a), P(dx), P(dw_ih), P(dw_hh), P(db_ih),
                  P(db_hh), P(da), P(dh0), P(dc0), P(ws), nbytes, T, B, D, H,
                  _lib.stream_of(x.device))
        if not f64:
            _poll(ws, x.device)
        return dx, dh0, dc0, dw_ih, dw_hh, db_ih, db_hh, da


class ParallelFn(torch.autograd.Function):
    """Parallel (scan) mode (``_parallel.py:38-74``).

    h0, W_hh, b_hh and a are accepted for the common signature but unused, so
    they receive no gradient (None), as in the reference.
    """

    @staticmethod
    def forward(ctx, x, h0, c0, w_ih, w_hh, b_ih, b_hh, a, eps):
        T, B, D, H = _check(x, h0, c0, w_ih, w_hh, b_ih, b_hh, a)
        x, c0, w_ih, b_ih = map(_c, (x, c0, w_ih, b_ih))
        ctx.set_materialize_grads(False)
        gates = x.new_empty(T, B, 4 * H)
        out = x.new_empty(T, B, H)
        c_ck = x.new_empty(_lib.load().hsl_scan_ck_rows(T), B, H)
        P = _lib.ptr
        _lib.call(_entry("hsl_par_fwd", x), P(x), P(c0), P(w_ih), P(b_ih), float(eps), P(gates), P(out),
                  P(c_ck), T, B, D, H, _lib.stream_of(x.device))
        ctx.save_for_backward(x, c0, w_ih, gates, c_ck)
        ctx.dims = (T, B, D, H)
        ctx.eps = float(eps)
        return out, out[T - 1], c_ck[-1]

    @staticmethod
    def backward(ctx, dout, dh_n, dc_n):
        x, c0, w_ih, gates, c_ck = ctx.saved_tensors
        T, B, D, H = ctx.dims
        dout = _c(dout) if dout is not None else x.new_zeros(T, B, H)
        dh_n, dc_n = _c(dh_n), _c(dc_n)
        need = ctx.needs_input_grad
        dx = torch.empty_like(x) if need[0] else None
        dc0 = x.new_empty(B, H) if need[2] else None
        dw_ih = torch.empty_like(w_ih)
        db_ih = x.new_empty(4 * H)
        lib = _lib.load()
        f64 = x.dtype == torch.float64
        nbytes = (lib.hsl_par_bwd_f64_ws_bytes if f64 else lib.hsl_par_bwd_ws_bytes)(T, B, D, H)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        P = _lib.ptr
        _lib.call(_entry("hsl_par_bwd", x), P(dout), P(dh_n), P(dc_n), P(x), P(c0), P(gates), P(c_ck),
                  P(w_ih), ctx.eps, P(dx), P(dw_ih), P(db_ih), P(dc0), P(ws), nbytes, T, B, D, H,
                  _lib.stream_of(x.device))
        return dx, None, dc0, dw_ih, None, db_ih, None, None, None


_HALF = (torch.bfloat16, torch.float16)


class ParallelHalfFn(torch.autograd.Function):
    """Parallel mode of a bf16/fp16 module: x and W_ih stay 16-bit for the input
    projection, which runs on 16-bit MFMA with fp32 accumulation (each product of two
    16-bit values is exact in fp32); c0 and b_ih arrive widened, and the scan and the
    whole backward compute in fp32, as in ``ParallelFn``.  The scan stores ``out`` in the
    module's 16-bit format (the rounding the module's output conversion would apply) and
    its backward reads the 16-bit ``dout`` as it is, so no [T,B,H] conversion pass runs
    either way; the backward also reads the 16-bit x and W_ih itself (``hsl_par_bwd_b16``,
    results equal to those on the widened operands)."""

    @staticmethod
    def forward(ctx, x, c0, w_ih, b_ih, eps):
        if x.dim() != 3:
            raise RuntimeError(f"x must be [T, B, D], got shape {tuple(x.shape)}")
        T, B, D = x.shape
        H = b_ih.shape[0] // 4
        if tuple(w_ih.shape) != (4 * H, D) or (c0 is not None and tuple(c0.shape) != (B, H)):
            raise RuntimeError("weight_ih_l0 must be [4H, D] and c0 [B, H]")
        for name, t in (("x", x), ("weight_ih_l0", w_ih), ("bias_ih_l0", b_ih), ("c0", c0)):
            if t is not None and (t.device.type != "cuda" or t.device != x.device):
                raise RuntimeError(f"prlstm_amd runs on ROCm devices only: {name} is on {t.device}")
        if w_ih.dtype != x.dtype or b_ih.dtype != torch.float32 or (c0 is not None and c0.dtype != torch.float32):
            raise RuntimeError("ParallelHalfFn: x and W_ih share a 16-bit dtype; b_ih and c0 are float32")
        x, c0, w_ih, b_ih = map(_c, (x, c0, w_ih, b_ih))
        ctx.set_materialize_grads(False)
        gates = x.new_empty(T, B, 4 * H, dtype=torch.float32)
        out = x.new_empty(T, B, H)  # the module's 16-bit format
        c_ck = x.new_empty(_lib.load().hsl_scan_ck_rows(T), B, H, dtype=torch.float32)
        fmt = 0 if x.dtype == torch.bfloat16 else 1
        P = _lib.ptr
        _lib.call("hsl_par_fwd_b16", P(x), P(c0), P(w_ih), P(b_ih), float(eps), P(gates), P(out),
                  P(c_ck), T, B, D, H, fmt, _lib.stream_of(x.device))
        ctx.save_for_backward(x, c0, w_ih, gates, c_ck)
        ctx.dims = (T, B, D, H)
        ctx.eps = float(eps)
        return out, out[T - 1], c_ck[-1]

    @staticmethod
    def backward(ctx, dout, dh_n, dc_n):
        x, c0, w_ih, gates, c_ck = ctx.saved_tensors
        T, B, D, H = ctx.dims
        # dout in out's 16-bit format (read as it is); dh_n and dc_n widened to fp32
        dout = _c(dout.to(x.dtype)) if dout is not None else x.new_zeros(T, B, H)
        dh_n = _c(dh_n.float()) if dh_n is not None else None
        dc_n = _c(dc_n.float()) if dc_n is not None else None
        need = ctx.needs_input_grad
        f32 = dict(device=x.device, dtype=torch.float32)
        dx = torch.empty(T, B, D, **f32) if need[0] else None
        dc0 = torch.empty(B, H, **f32) if need[1] else None
        dw_ih = torch.empty(4 * H, D, **f32)
        db_ih = torch.empty(4 * H, **f32)
        lib = _lib.load()
        nbytes = lib.hsl_par_bwd_b16_ws_bytes(T, B, D, H)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        P = _lib.ptr
        fmt = 0 if x.dtype == torch.bfloat16 else 1
        _lib.call("hsl_par_bwd_b16", P(dout), P(dh_n), P(dc_n), P(x), P(c0), P(gates), P(c_ck),
                  P(w_ih), ctx.eps, P(dx), P(dw_ih), P(db_ih), P(dc0), P(ws), nbytes, T, B, D, H, fmt,
                  _lib.stream_of(x.device))
        # autograd casts each gradient to its input's dtype (x and W_ih: 16-bit)
        return dx, dc0, dw_ih, db_ih, None


def _widen(args):
    """bf16/fp16 operands (a module moved with ``.to(dtype)``, as the reference's tests do for
    bf16, ``test_parallel.py:22-38``) are cast to fp32 here (recurrent mode; parallel mode
    keeps x and W_ih 16-bit for its projection, ``ParallelHalfFn``); the kernels then compute
    and accumulate in fp32 and the outputs are cast back.  The casts are autograd ops, so the
    gradients arrive in each operand's own dtype.  Returns (args, output dtype or None)."""
    dtype = args[0].dtype
    if dtype not in _HALF:
        return args, None
    return tuple(t.float() if torch.is_tensor(t) and t.dtype in _HALF else t for t in args), dtype


def _narrow(outs, dtype):
    return outs if dtype is None else tuple(t.to(dtype) for t in outs)


def headstartlstm_recurrent(x, h0, c0, W_ih, W_hh, b_ih, b_hh, a):
    """Recurrent-mode functional (drop-in for ``headstartlstm_torch``, ``_torch.py:173``)."""
    args, dtype = _widen((x, h0, c0, W_ih, W_hh, b_ih, b_hh, a))
    return _narrow(RecurrentFn.apply(*args), dtype)


def headstartlstm_parallel(x, h0, c0, W_ih, W_hh, b_ih, b_hh, a, eps=EPS):
    """Parallel-mode functional (drop-in for ``headstartlstm_parallel``, ``_parallel.py:38``)."""
    if x.dtype in _HALF and W_ih.dtype == x.dtype:  # 16-bit projection, fp32 everywhere else
        c0w = None if c0 is None else c0.float()
        return _narrow(ParallelHalfFn.apply(x, c0w, W_ih, b_ih.float(), eps), x.dtype)
    args, dtype = _widen((x, h0, c0, W_ih, W_hh, b_ih, b_hh, a))
    return _narrow(ParallelFn.apply(*args, eps), dtype)
