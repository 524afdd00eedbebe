"""The allocation-free apply (ifk_precondition_apply_bf16_noalloc) against the
workspace entry point it varies (ifk_precondition_apply_bf16), called through
the C ABI: two calls in a row, the second with a smaller input, each bit for
bit equal to the workspace entry's result (the library's scratch array has
room for the same split-K partials at these sizes); a warm call leaves the
device's free memory unchanged (it allocates nothing); and the size limit
rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inverse_copies(hip, n, seed):
    rng = np.random.default_rng(seed)
    R = np.triu(rng.standard_normal((n, n))) / np.sqrt(n) + 2 * np.eye(n)
    Rb = torch.tensor(R, dtype=torch.float32, device="cuda").to(torch.bfloat16)
    _, Zb, ZT = hip.tri_inverse_bf16(Rb)
    return Zb, ZT


def _noalloc(lib, g, ZX, ZG):
    nat = torch.empty(g.shape[0], g.shape[1], device="cuda")
    return _noalloc_into(lib, g, ZX, ZG, nat)


def _noalloc_into(lib, g, ZX, ZG, nat):
    n_out, n_in = g.shape
    rc = lib.ifk_precondition_apply_bf16_noalloc(
        torch.cuda.current_stream().cuda_stream, g.data_ptr(), n_out, n_in, g.stride(0),
        ZX[0].data_ptr(), ZX[1].data_ptr(), ZX[0].stride(0), ZG[0].data_ptr(), ZG[1].data_ptr(),
        ZG[0].stride(0), nat.data_ptr(), n_in)
    return rc, nat


def test_noalloc_apply_matches_workspace_entry(hip):
    from ifkfac_amd import _lib
    lib = _lib.load()
    out = []
    for n_out, n_in, seed in ((1100, 700, 1), (300, 257, 2)):   # the second call is smaller
        ZX = _inverse_copies(hip, n_in, seed)
        ZG = _inverse_copies(hip, n_out, seed + 10)
        g = torch.randn(n_out, n_in, device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(seed))
        rc, nat = _noalloc(lib, g, ZX, ZG)
        assert rc == 0, lib.ifk_last_error()
        want = hip.precondition_apply_bf16(g, ZX, ZG)
        torch.cuda.synchronize()
        assert torch.equal(nat, want), (n_out, n_in)
        out.append(nat)
    # the first result is unchanged by the second call (outputs are the caller's)
    assert out[0].shape == (1100, 700) and bool(torch.isfinite(out[0]).all())
    # a warm call allocates no device memory: the free memory the driver
    # reports (torch's cache aside, which this call does not touch) is the same
    # before and after
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    rc, _ = _noalloc_into(lib, g, ZX, ZG, nat)
    torch.cuda.synchronize()
    assert rc == 0, lib.ifk_last_error()
    assert torch.cuda.mem_get_info()[0] == free0


def test_noalloc_apply_rejects_sizes_beyond_the_scratch(hip):
    from ifkfac_amd import _lib
    lib = _lib.load()
    # 4096 x 4096 needs three 32 MiB bf16 buffers: more than the 64 MiB array.
    # Null pointers: the size check answers first, and the argument check
    # behind it would reject them too
    rc = lib.ifk_precondition_apply_bf16_noalloc(
        torch.cuda.current_stream().cuda_stream, None, 4096, 4096, 4096, None, None, 4096, None,
        None, 4096, None, 4096)
    assert rc == -1
    assert b"too large" in lib.ifk_last_error()
