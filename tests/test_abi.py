"""The C ABI library without a GPU: it loads, exports exactly what include/spanqr.h declares, and its host-side
pieces (dust generator, split policy, argument checks) behave; the product path refuses to run without the HIP
library or off the GPU (there is no CPU fallback)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import spanqr_amd
from spanqr_amd import _lib


def test_header_and_bindings_agree():
    assert set(_lib.exported_symbols_in_header()) == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _lib.exported_symbols_in_header() if not hasattr(L, n)]
    assert not missing


@pytest.mark.parametrize("K,r", [(7, 5), (300, 64), (1024, 256)])
def test_host_dust_is_the_oracle_dust(K, r):
    Z = np.empty((K, r), np.float32)
    _lib.check(_lib.lib().spanqr_dust_host(K, r, Z.ctypes.data_as(ctypes.c_void_p)))
    assert np.array_equal(Z.view(np.uint32), oracle.dust(K, r).view(np.uint32))


def test_split_policy():
    f = _lib.lib().spanqr_split_rows
    nparts = _lib.lib().spanqr_norm_partials
    # short X with many tiles (K <= 1024, r >= 448): two splits of ceil(K / 2) rows rounded up to 32, one norm partial per upper
    # 32x32 tile; otherwise tri.py:364-367 with 512 target workgroups: S = min(ceil(512 / U), ceil(K / 128)),
    # KS = 32 ceil(ceil(K/S) / 32), 16 partials per upper 64x64 tile
    for K, r in [(1024, 256), (2048, 256), (3584, 256), (768, 512), (2048, 512), (5120, 256), (17408, 256),
                 (64, 64), (100, 64), (12345, 192), (1024, 96), (4100, 160), (32, 32), (9217, 224), (768, 480),
                 (1024, 576), (2048, 768), (1100, 1024), (5000, 992), (1025, 512), (1024, 416), (512, 448),
                 (1024, 1024)]:
        nt = -(-r // 64)
        U = nt * (nt + 1) // 2
        if K <= 1024 and r >= 448:
            KS = 32 * -(-(-(-K // 2)) // 32)
            assert nparts(K, r) == (r // 32) * (r // 32 + 1) // 2, (K, r)
        else:
            S = max(1, min(-(-512 // U), -(-K // 128)))
            KS = 32 * -(-(-(-K // S)) // 32)
            assert KS % 32 == 0 and -(-K // KS) <= S
            assert nparts(K, r) == 16 * U, (K, r)
        assert f(K, r) == KS, (K, r)
    for K, r in [(100, 128), (1024, 80), (2048, 1056), (1024, 0), (4096, 1280), (1024, 16), (10, 32), (544, 576)]:
        assert f(K, r) == -1
        assert _lib.lib().spanqr_last_error()


def test_split_policy_is_the_oracle_rule():
    """the library's split rule (every Gram and block projection) is the one the oracle restates"""
    f = _lib.lib().spanqr_split_rows
    nparts = _lib.lib().spanqr_norm_partials
    for K in (64, 100, 513, 768, 1024, 1025, 2048, 3000, 17408, 65536):
        for r in range(32, 1025, 32):
            if K >= r:
                assert f(K, r) == oracle.gram_rows(K, r), (K, r)
                assert nparts(K, r) == oracle.npart_count(K, r), (K, r)
                assert (nparts(K, r) != 16 * (-(-r // 64)) * (-(-r // 64) + 1) // 2) == oracle.gram_short(K, r)


def test_column_blocked_shapes_checked_before_any_device_work():
    """spanqr_plan_create: column-blocked above 512 columns for multiples of 256 up to 4096, full-width kcholf for
    other multiples of 32 up to 1024; spanqr_plan_create_batched: full-width kcholf only (up to 1024 columns)"""
    h = ctypes.c_void_p()
    f = _lib.lib().spanqr_plan_create
    for K, r in [(1024, 1056), (2048, 1312), (512, 768), (8192, 4352), (1 << 19, 4096)]:
        assert f(K, r, 0, ctypes.byref(h)) == -1 and not h.value, (K, r)
    fb = _lib.lib().spanqr_plan_create_batched
    for K, r in [(2048, 1280), (4096, 2048), (1024, 1056), (512, 544)]:
        assert fb(K, r, 1, 0, ctypes.byref(h)) == -1 and not h.value, (K, r)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_column_blocked_plan_without_gpu_fails_cleanly():
    h = ctypes.c_void_p()
    assert _lib.lib().spanqr_plan_create(2048, 768, 0, ctypes.byref(h)) == -2 and not h.value


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU error path")
def test_plan_create_without_gpu_fails_cleanly():
    h = ctypes.c_void_p()
    rc = _lib.lib().spanqr_plan_create(1024, 256, 0, ctypes.byref(h))
    assert rc == -2 and not h.value
    assert _lib.lib().spanqr_last_error()


def test_borth_plan_arguments_checked_before_any_device_work():
    """spanqr_plan_create_borth (kbig.py:69's b and reorth): b a multiple of 32 in [32, 1024], r > b a multiple of b up
    to 4096, K >= r -- refused with SPANQR_EINVAL and no plan before any device call"""
    h = ctypes.c_void_p()
    f = _lib.lib().spanqr_plan_create_borth
    for K, r, b in [(1024, 1024, 96), (1024, 1024, 48), (1024, 1024, 16), (1024, 1024, 576), (1024, 512, 512),
                    (1024, 768, 512), (1000, 1024, 256), (8192, 8192, 512), (2048, 1024, 0), (4096, 2304, 1152),
                    (2048, 2048, 2048)]:
        assert f(K, r, b, 1, 0, ctypes.byref(h)) == -1 and not h.value, (K, r, b)
        assert _lib.lib().spanqr_last_error()
    assert f(1024, 1024, 256, 1, 0, None) == -1


def test_bad_shapes_rejected_before_any_device_work():
    h = ctypes.c_void_p()
    assert _lib.lib().spanqr_plan_create(100, 128, 0, ctypes.byref(h)) == -1
    assert _lib.lib().spanqr_plan_create(1024, 80, 0, ctypes.byref(h)) == -1     # r not a multiple of 32
    assert _lib.lib().spanqr_plan_create(2048, 1056, 0, ctypes.byref(h)) == -1   # above 1024, not a multiple of 256
    assert _lib.lib().spanqr_plan_create(1024, 256, 0, None) == -1


def test_batched_plan_arguments_checked_before_any_device_work():
    h = ctypes.c_void_p()
    f = _lib.lib().spanqr_plan_create_batched
    for batch in (0, -1, _lib.MAX_BATCH + 1):
        assert f(1024, 256, batch, 0, ctypes.byref(h)) == -1 and not h.value
        assert b"batch" in _lib.lib().spanqr_last_error()
    assert f(100, 128, 4, 0, ctypes.byref(h)) == -1
    assert f(1024, 256, 4, 0, None) == -1
    # a null plan is refused by the batched call as by the single one
    ptrs = (ctypes.c_void_p * 1)(None)
    assert _lib.lib().spanqr_orth_batched_f32(None, 1, ptrs, 256, ptrs, 256, 5e-7, 1e-7, 1e-8, 2, None) == -1


def test_orth_refuses_cpu_tensors():
    X = torch.randn(256, 128)
    with pytest.raises(TypeError):
        spanqr_amd.orth(X)
    with pytest.raises(TypeError):
        spanqr_amd.kcholqr_f(X)
    with pytest.raises(TypeError):
        spanqr_amd.orth(X.double())
    with pytest.raises(TypeError):
        spanqr_amd.orth_many([X, X])
    with pytest.raises(TypeError):
        spanqr_amd.kcholqr_f_many([X])
    with pytest.raises(TypeError):
        spanqr_amd.borth(torch.randn(1024, 768))
    assert spanqr_amd.orth_many([]) == [] and spanqr_amd.kcholqr_f_many([]) == []


def test_missing_library_raises(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libspanqr.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError):
        _lib.lib()


def test_top_level_orth_is_the_package_orth():
    import orth as top
    assert top.orth is spanqr_amd.orth
    assert top.orth_many is spanqr_amd.orth_many
    assert top.borth is spanqr_amd.borth and top.kcholqr_f is spanqr_amd.kcholqr_f


def test_chol64_arguments_checked_before_any_device_work():
    h = ctypes.c_void_p()
    f = _lib.lib().spanqr_chol64_plan_create
    for n in (0, 16, 48, 1056):
        assert f(n, 0, ctypes.byref(h)) == -1 and not h.value
    assert f(64, 0, None) == -1
    assert _lib.lib().spanqr_chol64(None, None, 64, None, None, None, None, None, None) == -1
    from spanqr_amd import kchol
    with pytest.raises(TypeError):
        kchol.chol64(torch.zeros(64, 64, dtype=torch.float64), 1e-9)
