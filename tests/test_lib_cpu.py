"""Host-side checks that need no GPU: the C ABI library, the module API surface."""

import ctypes
import re

import pytest
import torch
import torch.nn as nn

from conftest import ROOT
from oracle import hsl_oracle as O
import prlstm_amd
from prlstm_amd import _lib

HEADER = ROOT / "include" / "hsl.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hsl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = _declared()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares exactly the header's entry points
    assert sorted(_lib.SIGNATURES) == names


def test_abi_version_and_options():
    lib = _lib.load()
    assert lib.hsl_abi_version() == _lib.ABI_VERSION
    old = lib.hsl_set_recurrent_path(1)
    assert lib.hsl_set_recurrent_path(old) == 1
    prev = lib.hsl_set_spin_timeout_us(123)
    assert lib.hsl_set_spin_timeout_us(prev) == 123


def test_workspace_queries():
    lib = _lib.load()
    T, B, D, H = 256, 32, 256, 512
    fwd = lib.hsl_rec_fwd_ws_bytes(T, B, D, H)
    bwd = lib.hsl_rec_bwd_ws_bytes(T, B, D, H)
    if not torch.cuda.is_available():  # no device to plan on: sizes that cover every path
        assert fwd >= T * B * 4 * H * 4        # holds the input-gate buffer
        assert bwd >= T * B * 4 * H * 4        # holds dgates
        assert lib.hsl_rec_bwd_ws_bytes_for(T, B, D, H, 0) == bwd
    assert lib.hsl_rec_bwd_ws_bytes_for(T, B, D, H, 1) == bwd
    assert lib.hsl_rec_bwd_ws_bytes_for(T, B, D, H, 0) <= bwd
    assert lib.hsl_rec_fwd_ws_bytes(T, B, D, 2 * H) > fwd
    assert lib.hsl_par_bwd_ws_bytes(4096, 16, 256, 1024) >= 4096 * 16 * 4 * 1024 * 4
    assert lib.hsl_rec_fwd_ws_bytes(-1, 1, 1, 1) == 0
    assert lib.hsl_gemm_ws_bytes(2048, 512, 8192) > 0   # split-K for a long reduction
    assert lib.hsl_gemm_ws_bytes(8192, 2048, 256) == 0  # enough tiles: no split
    # fp64 modules: the recurrent workspaces hold the [T,B,4H] gates / dgates in fp64, the
    # parallel backward's its dgates; negative sizes give 0
    T, B, D, H = 256, 32, 256, 512
    assert lib.hsl_rec_fwd_f64_ws_bytes(T, B, D, H) >= T * B * 4 * H * 8
    assert lib.hsl_rec_bwd_f64_ws_bytes(T, B, D, H) >= T * B * 4 * H * 8
    assert lib.hsl_par_bwd_f64_ws_bytes(4096, 16, 256, 1024) >= 4096 * 16 * 4 * 1024 * 8
    for f in (lib.hsl_rec_fwd_f64_ws_bytes, lib.hsl_rec_bwd_f64_ws_bytes, lib.hsl_par_bwd_f64_ws_bytes):
        assert f(-1, 1, 1, 1) == 0
    # parallel mode keeps c every 8th step: ceil(T/8) carry-in rows, then c_n
    for T, rows in ((1, 2), (7, 2), (8, 2), (9, 3), (128, 17), (4096, 513), (0, 1), (-1, 0)):
        assert lib.hsl_scan_ck_rows(T) == rows, (T, lib.hsl_scan_ck_rows(T))


def test_argument_errors_are_reported_without_a_gpu():
    lib = _lib.load()
    rc = lib.hsl_rec_fwd(*([None] * 12), None, 0, -1, 1, 1, 1, None)
    assert rc == 1 and b"negative" in lib.hsl_last_error()
    rc = lib.hsl_gemm_f32(None, None, None, None, 4, 4, 4, 2, 4, 4, 0, 0, None, 0, None)
    assert rc == 1 and b"leading dimension" in lib.hsl_last_error()
    with pytest.raises(RuntimeError, match="hsl_rec_fwd failed"):
        _lib.call("hsl_rec_fwd", *([None] * 12), None, 0, 1, 1, 1, 1, None)
    # the fp64 entry points refuse null operands before any launch
    for name, args in (
            ("hsl_rec_fwd_f64", [None] * 13 + [0, 4, 2, 3, 5, None]),
            ("hsl_rec_bwd_f64", [None] * 21 + [0, 4, 2, 3, 5, None]),
            ("hsl_par_fwd_f64", [None] * 4 + [1e-6] + [None] * 3 + [4, 2, 3, 5, None]),
            ("hsl_par_bwd_f64", [None] * 8 + [1e-6] + [None] * 5 + [0, 4, 2, 3, 5, None])):
        assert getattr(lib, name)(*args) == 1, name
        assert b"null pointer" in lib.hsl_last_error(), (name, lib.hsl_last_error())


@pytest.mark.parametrize("T,B,D,H,why", [
    (1 << 16, 1 << 15, 8, 8, "T*B reaches 2^31 (GEMM rows, reduction length)"),
    (4, 2, 8, 1 << 15, "4H*H reaches 2^31 (the W_hh elements)"),
    (4, 2, 1 << 18, 2048, "4H*D reaches 2^31 (the W_ih elements)"),
    (4, 1 << 13, 8, 1 << 14, "one time step of [B, 4H] gates reaches 2^31 bytes"),
    (4, 1 << 12, 1 << 17, 8, "one time step of [B, D] inputs reaches 2^31 bytes"),
    (1 << 30, 1, 8, 8, "T reaches 2^30"),
])
def test_shapes_beyond_32_bit_indexing_are_rejected(T, B, D, H, why):
    """Every entry point that takes (T, B, D, H) refuses, before touching a pointer or the
    GPU, any shape whose sizes the kernels' and GEMMs' 32-bit index math cannot hold."""
    lib = _lib.load()
    calls = {
        "hsl_rec_fwd": lambda: lib.hsl_rec_fwd(*([None] * 12), None, 0, T, B, D, H, None),
        "hsl_rec_fwd_noalloc": lambda: lib.hsl_rec_fwd_noalloc(*([None] * 12), T, B, D, H, None),
        "hsl_rec_bwd": lambda: lib.hsl_rec_bwd(*([None] * 20), None, 0, T, B, D, H, None),
        "hsl_par_fwd": lambda: lib.hsl_par_fwd(None, None, None, None, 1e-6, None, None, None, T, B, D, H, None),
        "hsl_par_bwd": lambda: lib.hsl_par_bwd(*([None] * 8), 1e-6, None, None, None, None, None, 0,
                                               T, B, D, H, None),
        "hsl_rec_fwd_f64": lambda: lib.hsl_rec_fwd_f64(*([None] * 13), 0, T, B, D, H, None),
        "hsl_rec_bwd_f64": lambda: lib.hsl_rec_bwd_f64(*([None] * 21), 0, T, B, D, H, None),
        "hsl_par_fwd_f64": lambda: lib.hsl_par_fwd_f64(None, None, None, None, 1e-6, None, None, None,
                                                       T, B, D, H, None),
        "hsl_par_bwd_f64": lambda: lib.hsl_par_bwd_f64(*([None] * 8), 1e-6, None, None, None, None, None, 0,
                                                       T, B, D, H, None),
    }
    if D == 8:  # the scan entry points take no D
        calls["hsl_scan_fwd"] = lambda: lib.hsl_scan_fwd(None, None, 1e-6, None, None, T, B, H, None)
    for name, call in calls.items():
        rc = call()
        assert rc == 2, (name, why, rc, lib.hsl_last_error())  # HSL_ERR_UNSUPPORTED
        assert b"32-bit index range" in lib.hsl_last_error(), (name, lib.hsl_last_error())
    # the largest shapes of this build's configurations pass the check (they fail later,
    # on the null pointers, with HSL_ERR_ARG)
    assert lib.hsl_rec_fwd(*([None] * 12), None, 0, 64, 32, 1024, 2048, None) != 2


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libhsl.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()


def test_module_api_matches_reference():
    torch.manual_seed(0)
    m = prlstm_amd.HeadStartLSTM(16, 24)
    torch.manual_seed(0)
    r = O.RefHeadStartLSTM(16, 24)
    assert list(m.state_dict()) == ["weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0", "a"]
    for (n1, p1), (n2, p2) in zip(m.named_parameters(), r.named_parameters()):
        assert n1 == n2 and torch.equal(p1, p2)
    # same RNG consumption as nn.LSTM: the next draw agrees
    torch.manual_seed(1)
    prlstm_amd.HeadStartLSTM(8, 12)
    x1 = torch.randn(4)
    torch.manual_seed(1)
    nn.LSTM(8, 12)
    assert torch.equal(x1, torch.randn(4))
    # nn.LSTM weights load into the module (same names/shapes), plus `a`
    lstm = nn.LSTM(16, 24)
    sd = dict(lstm.state_dict())
    sd["a"] = torch.full((4,), 0.25)
    m.load_state_dict(sd)
    assert torch.equal(m.weight_hh_l0, lstm.weight_hh_l0) and float(m.a[2]) == 0.25
    m.set_mode(parallel=True)
    assert m.parallel
    with pytest.raises(AssertionError):
        prlstm_amd.HeadStartLSTM(4, 4, backend="cuda")
    for b in prlstm_amd.HeadStartLSTM._VALID_BACKENDS:
        prlstm_amd.HeadStartLSTM(4, 4, backend=b)


def test_cpu_tensors_are_rejected():
    m = prlstm_amd.HeadStartLSTM(8, 12)
    x = torch.randn(5, 3, 8)
    for parallel in (False, True):
        m.set_mode(parallel)
        with pytest.raises(RuntimeError, match="ROCm devices only"):
            m(x)


def test_shape_errors():
    H, D = 6, 5
    args = [torch.zeros(3, 2, D), torch.zeros(2, H), torch.zeros(2, H), torch.zeros(4 * H, D),
            torch.zeros(4 * H, H), torch.zeros(4 * H), torch.zeros(4 * H), torch.zeros(4)]
    bad = list(args)
    bad[3] = torch.zeros(4 * H, D + 1)
    with pytest.raises(RuntimeError, match="weight_ih_l0 must have shape"):
        prlstm_amd.headstartlstm_recurrent(*bad)
    bad = list(args)
    bad[7] = torch.zeros(3)
    with pytest.raises(RuntimeError, match="a must have shape"):
        prlstm_amd.headstartlstm_parallel(*bad)
