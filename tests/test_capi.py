"""The C ABI library loads on a host without a GPU and exports what the header declares.

No compute call is made here: only the version/size queries and argument
validation paths, which return before any launch.
"""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "ifkfac_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ifk_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from ifkfac_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from ifkfac_amd import build
        build.build()
    return _lib.load()


def test_header_declares_the_path():
    names = _declared_functions()
    for required in ("ifk_tsqr_fold", "ifk_finalize", "ifk_precondition", "ifk_precondition_apply",
                     "ifk_precondition_bias", "ifk_tri_inverse", "ifk_momentum_update",
                     "ifk_geqrf_r", "ifk_trsm", "ifk_potrf", "ifk_inv_spd", "ifk_last_error"):
        assert required in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    from ifkfac_amd import _lib
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(_declared_functions())


def test_version_and_sizes(lib):
    from ifkfac_amd import _lib
    assert lib.ifk_abi_version() == _lib.ABI_VERSION == 2
    assert lib.ifk_tsqr_fold_workspace_size(512, 1024) > 512 * 1024 * 4
    assert lib.ifk_finalize_workspace_size(1024) > 1024 * 1024 * 4
    assert lib.ifk_tri_inverse_workspace_size(11008) > 0
    assert lib.ifk_precondition_workspace_size(11008, 4096, 1) > 0
    assert lib.ifk_tsqr_fold_workspace_size(-1, 10) == 0


def test_invalid_arguments_are_rejected_before_launch(lib):
    r_out = ctypes.c_int64(0)
    # n = 0
    rc = lib.ifk_tsqr_fold(None, None, 0, 4, 0, 4, None, 4, 0, 0, None, 0, ctypes.byref(r_out))
    assert rc == -1
    assert b"invalid" in lib.ifk_last_error()
    # bad dtype code
    rc = lib.ifk_tsqr_fold(None, None, 7, 4, 4, 4, None, 4, 0, 0, None, 0, ctypes.byref(r_out))
    assert rc == -1
    # r_in > n
    rc = lib.ifk_finalize(None, None, 4, 0, 1.0, 0.1, None, 0, 4, 0, None, None, 0)
    assert rc == -1
    rc = lib.ifk_precondition(None, None, 0, 4, 4, None, 4, None, 4, 0, None, 4, 0, None, 0)
    assert rc == -1
    rc = lib.ifk_gemm(None, 0, 4, 4, 4, 1.0, None, 0, 2, 0, None, 0, 4, 0, 0.0, None, 4, None, 0)
    assert rc == -1  # lda < k


def test_cpu_tensor_is_refused():
    import torch
    from ifkfac_amd import IFKFACBackendError
    from ifkfac_amd._backend import HipBackend
    be = HipBackend()
    with pytest.raises(IFKFACBackendError):
        be.fold_(torch.zeros(4, 4), 0, torch.randn(8, 4), 0)
