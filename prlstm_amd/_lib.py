"""ctypes binding of libhsl.so (the C ABI declared in include/hsl.h).

The library is loaded on first use from this package directory.  A missing or
mismatched library raises RuntimeError: there is no fallback implementation.
"""

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libhsl.so"
ABI_VERSION = 3

_P = ctypes.c_void_p
_I = ctypes.c_int
_Z = ctypes.c_size_t
_F = ctypes.c_float
_D = ctypes.c_double

# name -> (restype, argtypes); must match include/hsl.h
SIGNATURES = {
    "hsl_abi_version": (_I, []),
    "hsl_last_error": (ctypes.c_char_p, []),
    "hsl_set_recurrent_path": (_I, [_I]),
    "hsl_set_spin_timeout_us": (ctypes.c_longlong, [ctypes.c_longlong]),
    "hsl_last_recurrent_path": (_I, []),
    "hsl_last_backward_fused": (_I, []),
    "hsl_set_exchange_scope": (_I, [_I]),
    "hsl_set_split_products": (_I, [_I]),
    "hsl_poll_error": (_I, [_P, _P, _P]),
    "hsl_device_errors": (_I, [_P, _I, _P]),
    "hsl_eval_math": (_I, [_I, _P, _P, _Z, _P]),
    "hsl_set_timing": (_I, [_I]),
    "hsl_timing_collect": (_I, [_I, _P, _P]),
    "hsl_rec_fwd_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_rec_fwd": (_I, [_P] * 12 + [_P, _Z, _I, _I, _I, _I, _P]),
    "hsl_rec_fwd_noalloc": (_I, [_P] * 12 + [_I, _I, _I, _I, _P]),
    "hsl_rec_bwd_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_rec_bwd_ws_bytes_for": (_Z, [_I, _I, _I, _I, _I]),
    "hsl_rec_bwd": (_I, [_P] * 20 + [_P, _Z, _I, _I, _I, _I, _P]),
    "hsl_par_fwd": (_I, [_P, _P, _P, _P, _F, _P, _P, _P, _I, _I, _I, _I, _P]),
    "hsl_par_fwd_b16": (_I, [_P, _P, _P, _P, _F, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "hsl_par_bwd_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_par_bwd": (_I, [_P] * 8 + [_F, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _P]),
    "hsl_par_bwd_b16_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_par_bwd_b16": (_I, [_P] * 8 + [_F, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _P]),
    "hsl_rec_fwd_f64_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_rec_fwd_f64": (_I, [_P] * 13 + [_Z, _I, _I, _I, _I, _P]),
    "hsl_rec_bwd_f64_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_rec_bwd_f64": (_I, [_P] * 20 + [_P, _Z, _I, _I, _I, _I, _P]),
    "hsl_par_fwd_f64": (_I, [_P, _P, _P, _P, _D, _P, _P, _P, _I, _I, _I, _I, _P]),
    "hsl_par_bwd_f64_ws_bytes": (_Z, [_I, _I, _I, _I]),
    "hsl_par_bwd_f64": (_I, [_P] * 8 + [_D, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _P]),
    "hsl_scan_ck_rows": (_I, [_I]),
    "hsl_scan_fwd": (_I, [_P, _P, _F, _P, _P, _I, _I, _I, _P]),
    "hsl_scan_bwd": (_I, [_P] * 6 + [_F, _P, _P, _P, _I, _I, _I, _P]),
    "hsl_gemm_ws_bytes": (_Z, [_I, _I, _I]),
    "hsl_gemm_f32": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "hsl_gemm_b16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load libhsl.so and declare every entry point; raises if it is unusable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m prlstm_amd.build` "
                "(prlstm_amd has no non-HIP fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)  # AttributeError = stale library
            fn.restype = res
            fn.argtypes = args
        v = lib.hsl_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libhsl ABI version {v}, expected {ABI_VERSION}; rebuild the library")
        _lib = lib
        return lib


def ptr(t):
    """Device pointer of a tensor (or NULL for None)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def call(name, *args):
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.hsl_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def set_recurrent_path(mode):
    """0 = automatic, 1 = one launch per time step, 2 = persistent only."""
    return load().hsl_set_recurrent_path(int(mode))


def set_split_products(on):
    """Large products and the persistent kernels' fused ones on split-bf16 MFMA (1, default)
    or on the fp32 instruction (0); returns the previous setting."""
    return load().hsl_set_split_products(1 if on else 0)


def set_exchange_scope(mode):
    """0 = automatic (XCD-local hand-off when verified), 1 = always device scope."""
    return load().hsl_set_exchange_scope(int(mode))


def set_spin_timeout_us(us):
    return load().hsl_set_spin_timeout_us(int(us))


def device_errors(device=None, clear=True):
    """The sticky device-error word of the current (or given) device; waits for its
    current stream.  Bit 0: a persistent kernel gave up a wait between workgroups."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    flags = ctypes.c_int(0)
    call("hsl_device_errors", ctypes.byref(flags), 1 if clear else 0, stream_of(dev))
    return flags.value


def check_errors(device=None):
    """Raise RuntimeError if a kernel of this library reported an error on the device
    since the last check (and clear it).  A persistent kernel that gives up a wait
    also leaves NaN in the outputs of that call, so the failure shows in the loss
    even without this check; this names it."""
    flags = device_errors(device, clear=True)
    if flags:
        raise RuntimeError(
            f"prlstm_amd: device error word {flags:#x}: a persistent recurrent kernel gave up a wait "
            "between workgroups (not all of its workgroups were resident at once, or a wait exceeded "
            "the spin timeout); the outputs of that call are NaN")


def last_recurrent_path():
    return load().hsl_last_recurrent_path()


def last_backward_fused():
    """0: weight gradients by separate GEMMs; 1: dW_hh, 2: dW_hh and dW_ih inside the
    persistent backward kernel (last backward in this process, any thread)."""
    return load().hsl_last_backward_fused()


TIMING_KINDS = {"rec_fwd": 1, "rec_bwd": 2, "scan_fwd": 3, "scan_bwd": 4, "input_proj": 5,
                "step_fwd": 6, "step_bwd": 7}


def set_timing(on):
    return load().hsl_set_timing(1 if on else 0)


def timing_collect(kind):
    """(total_ms, count) of the recorded launches of one kind (see include/hsl.h)."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int(0)
    call("hsl_timing_collect", int(TIMING_KINDS[kind]), ctypes.byref(ms), ctypes.byref(n))
    return ms.value, n.value
