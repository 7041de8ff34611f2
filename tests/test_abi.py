"""The C-ABI library (libgfl_moe.so) loads, exports every entry point include/gfl_moe.h declares, and its host-side
logic behaves; no GPU needed (device entry points are only called for their argument checks)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "gfl_moe.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gfl_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import _native
    return _native.load()


def test_library_exports_every_declared_symbol(lib):
    import _native
    syms = header_symbols()
    assert len(syms) >= 12
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (gfl_[a-z_0-9]+)", out))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    assert set(syms) == set(_native.SYMBOLS)
    for s in syms:
        getattr(lib, s)
    # every entry point with arguments is typed for ctypes (an untyped float or int64 argument would be mangled)
    untyped = [s for s in syms if s not in ("gfl_last_error", "gfl_version") and getattr(lib, s).argtypes is None]
    assert not untyped, untyped


def test_version_and_error_string(lib):
    assert lib.gfl_version() == 101
    assert isinstance(lib.gfl_last_error(), bytes)


def test_argument_checks_without_device(lib):
    import _native
    # NULL context / NULL pointers are rejected before any device work
    assert lib.gfl_moe_forward(None, 0, None, None, None, 0, 1, 8, None, 1, 0.0, None) == 1
    assert b"NULL" in lib.gfl_last_error()
    assert lib.gfl_dequant(None, 16, 16, 3, None, None) == 1
    assert lib.gfl_register_layer(None, 0, 1, 128, 128, 3, 3, 3, None) == 1
    assert lib.gfl_split(*([None] * 3), 1, 8, 8, 8, 0, *([None] * 6), 0, 0, 0, *([None] * 5), None) == 1
    assert lib.gfl_combine(None, 0, 1, None, None, None, None, 0, None) == 1
    with pytest.raises(_native.NativeError):
        _native.check(lib.gfl_stats(None, None, 0))
    assert lib.gfl_ctx_set_shared(None, 1) == 1
    assert b"gfl_ctx_set_shared" in lib.gfl_last_error()
    assert lib.gfl_ctx_check(None) == 1 and b"NULL" in lib.gfl_last_error()
    assert lib.gfl_ingress_serve(None, 0, 1, 8, None, None, None, None, -1, 0.0, None) == 1
    assert lib.gfl_register_shared(None, 0, 3, 3, 3, None) == 1 and b"NULL" in lib.gfl_last_error()
    assert lib.gfl_moe_forward_shared(None, 0, None, None, None, 0, 1, 8, None, 1, 0.0, None) == 1


def test_grouped_rows_host_matches_oracle(oracle):
    import _native
    rng = np.random.default_rng(12)
    T, K, E = 17, 8, 48
    sel = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int64)
    sel[3, 2] = -1
    w = rng.random((T, K)).astype(np.float32)
    w[3, 2] = 0
    take = (rng.random(E) < 0.6).astype(np.uint8)
    a = _native.grouped_rows(sel, w, take, E)
    b = oracle.grouped_rows(sel, w, take, E)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    dup = sel.copy(); dup[0, 1] = dup[0, 0]
    with pytest.raises(ValueError, match="duplicate"):
        _native.grouped_rows(dup, w, np.ones(E, np.uint8), E)
    badt = np.ones(E, np.uint8); badt[3] = 2
    with pytest.raises(ValueError, match="zero or one"):
        _native.grouped_rows(sel, w, badt, E)


def test_missing_library_fails_loudly(tmp_path):
    import _native
    with pytest.raises(_native.NativeUnavailable):
        saved = _native._LIB
        _native._LIB = None
        try:
            _native.load(str(tmp_path / "absent.so"))
        finally:
            _native._LIB = saved


def test_silu_table_is_the_fp32_gate():
    """The device's gate table equals g / (1 + expf(-g)) with one fp32 rounding per operation (silu, ft_core.h:123) at
    every fp16 input, including the signed zeros, infinities (-inf gives NaN) and the underflow to -0 for large
    negative g."""
    import _native
    tab = _native.silu_table()
    e = _native.exp_table()
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    with np.errstate(all="ignore"):
        want = g / (np.float32(1.0) + e)
    assert want.dtype == np.float32
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(tab), nan)
    assert np.array_equal(tab[~nan].view(np.uint32), want[~nan].view(np.uint32))
    f16 = lambda v: int(np.array([v], np.float16).view(np.uint16)[0])
    assert tab[f16(0.0)] == 0.0 and tab[f16(np.inf)] == np.inf and np.isnan(tab[f16(-np.inf)])
    big = tab[f16(-60000.0)]
    assert big == 0.0 and np.signbit(big)
    assert abs(tab[f16(1.0)] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-7


def test_exp_table_is_the_c_library_expf():
    """The activation's exponential table equals the C library's expf at every fp16 input (what silu calls,
    ft_core.h:123). It also documents why a table is used: correctly rounded exp disagrees with it on some inputs."""
    import ctypes as C
    import math
    import _native
    tab = _native.exp_table()
    libm = C.CDLL("libm.so.6")
    libm.expf.restype, libm.expf.argtypes = C.c_float, [C.c_float]
    g = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    want = np.array([libm.expf(float(-v)) for v in g], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(tab), nan)
    assert np.array_equal(tab[~nan].view(np.uint32), want[~nan].view(np.uint32))
    fin = np.isfinite(g) & (np.abs(g) < 80)
    cr = np.array([np.float32(math.exp(float(-v))) for v in g[fin]], np.float32)
    assert (cr.view(np.uint32) != want[fin].view(np.uint32)).sum() > 0


def test_forward_width_check_without_device():
    """Context refuses x whose width differs from the registered layer's H before calling into the library (host
    logic only: a Context shell with a recorded layer shape, no device)."""
    import torch
    import _native
    ctx = object.__new__(_native.Context)
    ctx.h, ctx.device, ctx._keep, ctx._shape = None, 0, {}, {3: (8, 512, 256, 3, 3, 3)}
    ctx._check_width(3, torch.zeros((2, 512), dtype=torch.float16))
    for width in (256, 1024):
        with pytest.raises(ValueError, match="H = 512"):
            ctx._check_width(3, torch.zeros((2, width), dtype=torch.float16))
