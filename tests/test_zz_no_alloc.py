"""The allocation-free apply (ifk_precondition_apply_bf16_noalloc) against the
workspace entry point it varies (ifk_precondition_apply_bf16), called through
the C ABI: two calls in a row, the second with a smaller input, each bit for
bit equal to the workspace entry's result (the library's scratch array has
room for the same split-K partials at these sizes), and the size limit
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
    n_out, n_in = g.shape
    nat = torch.empty(n_out, n_in, device="cuda")
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


def test_noalloc_apply_rejects_sizes_beyond_the_scratch(hip):
    from ifkfac_amd import _lib
    lib = _lib.load()
    # 4096 x 4096 needs three 32 MiB bf16 buffers: more than the 64 MiB array
    rc = lib.ifk_precondition_apply_bf16_noalloc(
        torch.cuda.current_stream().cuda_stream, 1, 4096, 4096, 4096, 1, 1, 4096, 1, 1, 4096, 1,
        4096)
    assert rc == -1
    assert b"too large" in lib.ifk_last_error()
