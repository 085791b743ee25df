"""hsl_rec_fwd_noalloc, the forward entry point that allocates nothing (its workspace is
a static scratch array in the library), against hsl_rec_fwd with a caller-allocated
workspace: two calls in a row, the second with a smaller input, must give the same
h_save, c_save, gact and tanh_c bit for bit (the same kernels run on the same path); the
call is replayed from a captured HIP graph with fresh inputs; repeated calls leave the
device's free memory unchanged; a shape whose workspace exceeds the scratch is rejected
before any work is enqueued."""

import pytest
import torch

from prlstm_amd import _lib

pytestmark = pytest.mark.gpu

NOALLOC_SCRATCH_BYTES = 4 << 20  # the static scratch array of hsl_rec_fwd_noalloc


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


def _reference(i, T, B, D, H, dev):
    """hsl_rec_fwd on the same inputs with a caller-allocated workspace."""
    lib = _lib.load()
    ref = _outputs(T, B, H, dev)
    nbytes = lib.hsl_rec_fwd_ws_bytes(T, B, D, H)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    _lib.call("hsl_rec_fwd", *_args(i, ref), _lib.ptr(ws), nbytes, T, B, D, H, _lib.stream_of(dev))
    torch.cuda.synchronize()
    return ref


def _assert_equal(got, ref, what):
    for n in ref:
        assert torch.isfinite(got[n]).all(), (what, n)
        assert torch.equal(got[n], ref[n]), (what, n)


def test_rec_fwd_noalloc_matches_workspace_entry_point(dev):
    s = _lib.stream_of(dev)
    for T, B, D, H in [(256, 32, 256, 512), (40, 12, 64, 128)]:
        print(f"noalloc T={T} B={B} D={D} H={H}", flush=True)
        i = _inputs(T, B, D, H, dev, seed=T + H)
        ref = _reference(i, T, B, D, H, dev)
        got = _outputs(T, B, H, dev)
        _lib.call("hsl_rec_fwd_noalloc", *_args(i, got), T, B, D, H, s)
        torch.cuda.synchronize()
        assert _lib.last_recurrent_path() == 2
        _assert_equal(got, ref, f"T={T}")
    _lib.check_errors(dev)


def test_rec_fwd_noalloc_keeps_free_memory_flat(dev):
    """Repeated eager calls allocate nothing: the device's free memory does not move."""
    T, B, D, H = 64, 32, 256, 512
    i = _inputs(T, B, D, H, dev, seed=7)
    o = _outputs(T, B, H, dev)
    s = _lib.stream_of(dev)
    _lib.call("hsl_rec_fwd_noalloc", *_args(i, o), T, B, D, H, s)  # first call: symbol address, code load
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(dev)[0]
    for _ in range(5):
        _lib.call("hsl_rec_fwd_noalloc", *_args(i, o), T, B, D, H, s)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free0
    _lib.check_errors(dev)


def test_rec_fwd_noalloc_under_graph_capture(dev):
    """One eager call, then the call captured in a HIP graph; every replay, on new inputs
    copied into the captured buffers and with eager work between replays, equals
    hsl_rec_fwd on those inputs bit for bit."""
    T, B, D, H = 96, 32, 256, 512
    st = _inputs(T, B, D, H, dev, seed=11)
    so = _outputs(T, B, H, dev)
    _lib.call("hsl_rec_fwd_noalloc", *_args(st, so), T, B, D, H, _lib.stream_of(dev))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.call("hsl_rec_fwd_noalloc", *_args(st, so), T, B, D, H, _lib.stream_of(dev))
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        new = _inputs(T, B, D, H, dev, seed=100 + rep)
        for n in st:
            st[n].copy_(new[n])
        for n in so:
            so[n].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        ref = _reference(new, T, B, D, H, dev)  # eager work between the replays
        _assert_equal(so, ref, f"replay {rep}")
    _lib.check_errors(dev)


def test_rec_fwd_noalloc_rejects_shapes_beyond_its_scratch(dev):
    """configs[3] (H=2048) runs the W_hh-resident wide kernels, whose workspace (the
    [T,B,4H] input-gate buffer alone is 32 MiB) is far beyond the 4 MiB scratch: the call,
    given real buffers of the right sizes, refuses before enqueuing anything."""
    T, B, D, H = 64, 32, 1024, 2048
    lib = _lib.load()
    assert lib.hsl_rec_fwd_ws_bytes(T, B, D, H) > NOALLOC_SCRATCH_BYTES
    i = _inputs(T, B, D, H, dev, seed=3)
    o = _outputs(T, B, H, dev)
    torch.cuda.synchronize()
    rc = lib.hsl_rec_fwd_noalloc(*_args(i, o), T, B, D, H, _lib.stream_of(dev))
    assert rc == 2, rc  # HSL_ERR_UNSUPPORTED
    assert b"static scratch" in lib.hsl_last_error()
    torch.cuda.synchronize()
    for n in o:  # nothing ran: the outputs still hold their NaN fill
        assert torch.isnan(o[n]).all(), n
