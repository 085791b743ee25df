"""hsl_rec_fwd_noalloc, the forward entry point that allocates nothing (its workspace is
a static scratch array in the library), against hsl_rec_fwd with a caller-allocated
workspace: two calls in a row, the second with a smaller input, must give the same
h_save, c_save, gact and tanh_c bit for bit (the same kernels run on the same path); a
shape whose workspace exceeds the scratch is rejected before any work is enqueued."""

import ctypes

import pytest
import torch

from prlstm_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(T, B, D, H, dev, seed):
    g = torch.Generator().manual_seed(seed)
    k = H ** -0.5
    t = {
        "x": torch.randn(T, B, D, generator=g),
        "h0": 0.5 * torch.randn(B, H, generator=g),
        "c0": 0.5 * torch.randn(B, H, generator=g),
        "w_ih": (torch.rand(4 * H, D, generator=g) * 2 - 1) * k,
        "w_hh": (torch.rand(4 * H, H, generator=g) * 2 - 1) * k,
        "b_ih": (torch.rand(4 * H, generator=g) * 2 - 1) * k,
        "b_hh": (torch.rand(4 * H, generator=g) * 2 - 1) * k,
        "a": torch.rand(4, generator=g) * 0.5,
    }
    return {n: v.to(dev) for n, v in t.items()}


def _outputs(T, B, H, dev):
    return {"h_save": torch.full((T + 1, B, H), float("nan"), device=dev),
            "c_save": torch.full((T + 1, B, H), float("nan"), device=dev),
            "gact": torch.full((T, B, H, 4), float("nan"), device=dev),
            "tanh_c": torch.full((T, B, H), float("nan"), device=dev)}


def _args(i, o):
    P = _lib.ptr
    return [P(i[n]) for n in ("x", "h0", "c0", "w_ih", "w_hh", "b_ih", "b_hh", "a")] + \
           [P(o[n]) for n in ("h_save", "c_save", "gact", "tanh_c")]


def test_rec_fwd_noalloc_matches_workspace_entry_point(dev):
    lib = _lib.load()
    s = _lib.stream_of(dev)
    for T, B, D, H in [(256, 32, 256, 512), (40, 12, 64, 128)]:
        print(f"noalloc T={T} B={B} D={D} H={H}", flush=True)
        i = _inputs(T, B, D, H, dev, seed=T + H)
        ref = _outputs(T, B, H, dev)
        nbytes = lib.hsl_rec_fwd_ws_bytes(T, B, D, H)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
        _lib.call("hsl_rec_fwd", *_args(i, ref), _lib.ptr(ws), nbytes, T, B, D, H, s)
        got = _outputs(T, B, H, dev)
        _lib.call("hsl_rec_fwd_noalloc", *_args(i, got), T, B, D, H, s)
        torch.cuda.synchronize()
        assert _lib.last_recurrent_path() == 2
        for n in ref:
            assert torch.isfinite(got[n]).all(), n
            assert torch.equal(got[n], ref[n]), n
    _lib.check_errors(dev)


def test_rec_fwd_noalloc_rejects_shapes_beyond_its_scratch(dev):
    """configs[3] (H=2048) runs one launch per step and needs its [T,B,4H] gate buffer and
    the 64 MiB rearranged W_hh: far beyond the scratch, so the call refuses up front."""
    T, B, D, H = 64, 32, 1024, 2048
    lib = _lib.load()
    rc = lib.hsl_rec_fwd_noalloc(*([ctypes.c_void_p(16)] * 12), T, B, D, H, _lib.stream_of(dev))
    assert rc == 2, rc  # HSL_ERR_UNSUPPORTED
    assert b"static scratch" in lib.hsl_last_error()
