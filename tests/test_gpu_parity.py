"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Tolerances (stated per test):
  factors   ||R^T R - R_o^T R_o||_F / ||R_o^T R_o||_F <= 4 * kappa(R_o) * eps(storage)
            (fp32 eps = 1.19e-7).  For bf16 arithmetic the stated bound
            4 kappa eps_bf16 is vacuous at kappa ~ 1e2, so the test also holds
            the result to a tighter measured regression bound.
  nat grad  relative error <= 1e-5 (fp32 mode), <= 2e-2 (bf16 mode), against the
            oracle's solves on the same factors.
Inputs are seeded; the kappa-controlled matrices use U diag(s) V^T with Haar
U, V and log-spaced s (tests/test_bf16_stability.py:23-29 of the reference).
"""
import math

import numpy as np
import pytest
import torch

from oracle import ifk_oracle as O

pytestmark = pytest.mark.gpu

EPS32 = 1.1920929e-07
EPS_BF16 = 7.8125e-03
DEV = "cuda"


def _gram_rel(R, Ro):
    R = R.double().cpu().numpy() if isinstance(R, torch.Tensor) else R
    a = R.T @ R
    b = Ro.T @ Ro
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def _kappa(Ro):
    s = np.linalg.svd(Ro, compute_uv=False)
    return s[0] / max(s[-1], 1e-300)


def _rel(a, b):
    a = a.double().cpu().numpy() if isinstance(a, torch.Tensor) else a
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


# --------------------------------------------------------------------------- GEMM engine


@pytest.mark.parametrize("math_", [0, 1])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (200, 130, 77), (64, 1000, 4096), (1, 37, 1000)])
def test_gemm_engine(hip, math_, ta, tb, m, n, k):
    g = torch.Generator(device=DEV).manual_seed(m * 7 + n + k)
    A = torch.randn((k, m) if ta else (m, k), device=DEV, generator=g)
    B = torch.randn((n, k) if tb else (k, n), device=DEV, generator=g).to(torch.bfloat16)
    opA = A.t() if ta else A
    opB = B.t() if tb else B
    if math_ == 1:
        ref = opA.bfloat16().double() @ opB.double()
    else:
        ref = opA.double() @ opB.double()
    C = hip.gemm(A, B, ta, tb, math_)
    assert _rel(C, ref.cpu().numpy()) < 2e-6


@pytest.mark.parametrize("adt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("m,n,k", [(1100, 900, 1100), (700, 1300, 1500), (2048, 2560, 512)])
def test_gemm_engine_large_tiles(hip, adt, ta, tb, m, n, k):
    """Shapes that take the 256 x 256 bf16 kernel (ragged edges, split-K for
    the first two, full tiles for the last), against an fp64 product of the
    bf16-rounded operands."""
    g = torch.Generator(device=DEV).manual_seed(m + 3 * n + 7 * k)
    A = torch.randn((k, m) if ta else (m, k), device=DEV, generator=g).to(adt)
    B = torch.randn((n, k) if tb else (k, n), device=DEV, generator=g).to(adt)
    opA = A.t() if ta else A
    opB = B.t() if tb else B
    ref = opA.bfloat16().double() @ opB.bfloat16().double()
    C = hip.gemm(A, B, ta, tb, 1)
    assert _rel(C, ref.cpu().numpy()) < 2e-6


@pytest.mark.parametrize("m,n,k", [(2048, 2560, 512), (600, 520, 4096), (1000, 700, 2048),
                                   (512, 512, 8192), (256, 384, 16384), (4000, 3700, 256),
                                   (3840, 3840, 1024)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gemm_direct_lds_kernel(hip, m, n, k, beta):
    """bf16 operands with K contiguous take the direct-to-LDS kernel (its 128
    tile below 224 tiles of 256, its 256 tile from there: the last two
    shapes): ragged M and N (rows past the operand read as zero through the
    buffer bounds), split-K for few tiles, alpha / beta, against an fp64
    product."""
    g = torch.Generator(device=DEV).manual_seed(m + 5 * n + 3 * k)
    A = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    B = torch.randn(n, k, device=DEV, generator=g).to(torch.bfloat16)
    C0 = torch.randn(m, n, device=DEV, generator=g)
    ref = -0.5 * (A.double() @ B.double().t()) + beta * C0.double()
    C = hip.gemm(A, B, False, True, 1, -0.5, beta, C0.clone())
    assert _rel(C, ref.cpu().numpy()) < 2e-6


@pytest.mark.parametrize("m,n,k", [(1000, 701, 2048), (4000, 3701, 256)])
@pytest.mark.parametrize("ldc_pad", [0, 3])
def test_gemm_direct_lds_epilogue(hip, m, n, k, ldc_pad):
    """The direct-to-LDS kernel's output paths: with C rows 16-byte aligned
    (ld a multiple of 4, here n + 3) the epilogue goes through LDS and writes
    four columns per lane, the last partial group element by element; with
    ld = n it writes element by element.  Both tiles, beta = 1."""
    g = torch.Generator(device=DEV).manual_seed(m + n + k + ldc_pad)
    A = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    B = torch.randn(n, k, device=DEV, generator=g).to(torch.bfloat16)
    buf = torch.randn(m, n + ldc_pad, device=DEV, generator=g)
    pad = buf[:, n:].clone()
    C0 = buf[:, :n]
    ref = 0.75 * (A.double() @ B.double().t()) + C0.double()
    C = hip.gemm(A, B, False, True, 1, 0.75, 1.0, C0)
    assert C.data_ptr() == buf.data_ptr() and C.stride(0) == n + ldc_pad
    assert _rel(C, ref.cpu().numpy()) < 2e-6
    assert torch.equal(buf[:, n:], pad)   # the columns past n are untouched


def _gemm_variants(fn):
    """Run fn with the GEMM launch profiler armed for every variant; returns
    (fn's result, [(variant, m, n, k), ...])."""
    import ctypes
    from ifkfac_amd import _lib
    lib = _lib.load()
    torch.cuda.synchronize()
    _lib.check(lib.ifk_profile_begin(-2), "profile_begin")
    try:
        out = fn()
        torch.cuda.synchronize()
    finally:
        cnt = ctypes.c_int64(0)
        _lib.check(lib.ifk_profile_end(ctypes.byref(cnt)), "profile_end")
    v, ms, fl, by = ctypes.c_int(), ctypes.c_float(), ctypes.c_double(), ctypes.c_double()
    m_, n_, k_ = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    res = []
    for i in range(cnt.value):
        _lib.check(lib.ifk_profile_get(i, *(ctypes.byref(x) for x in (v, ms, fl, by, m_, n_, k_))),
                   "profile_get")
        res.append((v.value, m_.value, n_.value, k_.value))
    return out, res


@pytest.mark.parametrize("m,n,k", [(9984, 1024, 16384), (10000, 1000, 16000), (9000, 777, 12000),
                                   (3000, 1000, 9000)])
@pytest.mark.parametrize("beta", [0.0, 1.0])
def test_gemm_stream_k(hip, m, n, k, beta):
    """Plain bf16 products with few output tiles and a long K (the Gram
    route's Gram columns: N = 1024, K = p; ragged edges; the last on the 128
    tile) take the stream-K walk of the direct-to-LDS kernel: against an
    fp64 product of the same bf16 operands at 2e-6, and bit for bit equal on
    a second call (a shared tile's shares are summed in lane order, whatever
    order they arrive in)."""
    g = torch.Generator(device=DEV).manual_seed(m + 11 * n + 3 * k)
    A = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    B = torch.randn(n, k, device=DEV, generator=g).to(torch.bfloat16)
    C0 = torch.randn(m, n, device=DEV, generator=g)
    ref = 0.5 * (A.double() @ B.double().t()) + beta * C0.double()
    C1, var = _gemm_variants(lambda: hip.gemm(A, B, False, True, 1, 0.5, beta, C0.clone()))
    C2 = hip.gemm(A, B, False, True, 1, 0.5, beta, C0.clone())
    assert len(var) == 1 and (var[0][0] >> 9) & 1 and (var[0][0] >> 6) & 1
    assert _rel(C1, ref.cpu().numpy()) < 2e-6
    assert torch.equal(C1, C2)


@pytest.mark.parametrize("tri", ["upper_a", "lower_a", "lower_b", "upper_b"])
@pytest.mark.parametrize("n,rows", [(1280, 1100), (4096, 3600), (2900, 5000), (11008, 300)])
def test_gemm_direct_lds_triangular(hip, tri, n, rows):
    """Triangular bf16 operands (as in the preconditioner) through the
    direct-to-LDS kernel, both tiles and the XCD walks over ragged tile
    counts: the stored zero triangle is filled with garbage, which the kernel
    must ignore."""
    g = torch.Generator(device=DEV).manual_seed(42)
    Z = torch.randn(n, n, device=DEV, generator=g)
    G = torch.randn(rows, n, device=DEV, generator=g).to(torch.bfloat16)
    Zt = torch.triu(Z).to(torch.bfloat16)
    noisy = (Zt.float() + torch.tril(torch.randn(n, n, device=DEV, generator=g), -1)).to(
        torch.bfloat16)
    if tri == "upper_a":
        # C = U G^T: op(A) = U upper triangular, B = G stored (n_rows x K)
        ref = Zt.double() @ G.double().t()
        C = hip.gemm(noisy, G, False, True, 1, tri_a=1)
    elif tri == "lower_a":
        # C = L G^T: op(A) = L = U^T lower triangular, given row-major,
        # garbage above its diagonal
        ref = Zt.double().t() @ G.double().t()
        noisyT = (Zt.float().t() + torch.triu(torch.randn(n, n, device=DEV, generator=g), 1)).to(
            torch.bfloat16).contiguous()
        C = hip.gemm(noisyT, G, False, True, 1, tri_a=2)
    elif tri == "lower_b":
        # C = G U^T: op(B) = U^T lower triangular, given as B[n][k] = U
        ref = G.double() @ Zt.double().t()
        C = hip.gemm(G, noisy, False, True, 1, tri_b=2)
    else:
        # C = G U: op(B) = U upper triangular, given as B[n][k] = U^T (the
        # layout of the fold's T^T), garbage above its diagonal
        ref = G.double() @ Zt.double()
        noisyT = (Zt.float().t() + torch.triu(torch.randn(n, n, device=DEV, generator=g), 1)).to(
            torch.bfloat16).contiguous()
        C = hip.gemm(G, noisyT, False, True, 1, tri_b=1)
    assert _rel(C, ref.cpu().numpy()) < 2e-6


# --------------------------------------------------------------------------- fold


def _fold_chunks(hip, chunks, n, math_=0):
    R = torch.zeros(n, n, device=DEV)
    r = 0
    for X in chunks:
        r = hip.fold_(R, r, X, math_)
    return R, r


@pytest.mark.parametrize("chunks,n", [
    ([256], 128), ([256], 256), ([256], 10),            # demo MLP layer shapes
    ([64, 64], 40), ([30, 30, 100], 50), ([5, 7, 3], 20),  # trapezoid growth
    ([300], 200), ([2000], 256), ([1, 1, 1], 2), ([1], 1),
    ([512] * 3, 1024), ([100, 1000], 333),
    # several outer blocks, so the far columns run on the helper stream
    ([3000], 1600), ([700, 2500], 1600), ([400, 300], 1700), ([1200, 1200], 2100),
])
def test_fold_matches_oracle_fp32(hip, chunks, n):
    g = torch.Generator(device=DEV).manual_seed(sum(chunks) + n)
    Xs = [torch.randn(p, n, device=DEV, generator=g) for p in chunks]
    R, r = _fold_chunks(hip, Xs, n)
    Ro = None
    for X in Xs:
        Ro = O.streaming_tsqr_update(Ro, X.double().cpu().numpy())
    assert r == Ro.shape[0]
    Rg = R[:r].double().cpu().numpy()
    assert np.all(np.diag(Rg) >= 0)
    assert np.array_equal(np.tril(Rg, -1), np.zeros_like(np.tril(Rg, -1)))
    assert torch.count_nonzero(R[r:]).item() == 0
    if r == n:
        kap = _kappa(Ro)
        assert _gram_rel(Rg, Ro) <= 4 * kap * EPS32
        assert np.abs(Rg - Ro).max() / np.abs(Ro).max() < 1e-4
    else:  # trapezoid: compare the rows directly
        assert np.abs(Rg - Ro).max() / np.abs(Ro).max() < 1e-4


def test_fold_rank_deficient_and_zero_columns(hip):
    g = torch.Generator(device=DEV).manual_seed(11)
    X = torch.randn(100, 30, device=DEV, generator=g)
    X[:, 5] = 0
    X[:, 17] = 0
    X[:, 20] = X[:, 3]          # duplicated column
    R, r = _fold_chunks(hip, [X], 30)
    Xd = X.double().cpu().numpy()
    G = Xd.T @ Xd
    Rg = R.double().cpu().numpy()
    assert np.linalg.norm(Rg.T @ Rg - G) / np.linalg.norm(G) < 1e-6


@pytest.mark.parametrize("seed", range(6))
def test_fold_rows_summing_to_zero(hip, seed):
    """Output-layer deltas of a softmax cross-entropy (softmax - onehot) sum to
    zero over the classes, so a 256 x 10 chunk has rank 9.  Two chunks are
    folded in turn (the second onto a full R, as on every later step): the
    running R must keep R^T R = sum X_i^T X_i and match the oracle on its
    leading full-rank rows."""
    g = torch.Generator(device=DEV).manual_seed(100 + seed)
    chunks = []
    for _ in range(2):
        logits = torch.randn(256, 10, device=DEV, generator=g) * 2
        onehot = torch.nn.functional.one_hot(
            torch.randint(0, 10, (256,), device=DEV, generator=g), 10).float()
        chunks.append((torch.softmax(logits, -1) - onehot) / 256)
    R = torch.zeros(10, 10, device=DEV)
    r = 0
    G = np.zeros((10, 10))
    R_or = None
    for X in chunks:
        r = hip.fold_(R, r, X, 0)
        Xd = X.double().cpu().numpy()
        G += Xd.T @ Xd
        R_or = O.streaming_tsqr_update(R_or, Xd)
        Rg = R.double().cpu().numpy()
        assert np.linalg.norm(Rg.T @ Rg - G) / np.linalg.norm(G) < 1e-5
        assert np.abs(Rg[:9] - R_or[:9]).max() / np.abs(R_or).max() < 1e-4


@pytest.mark.parametrize("kappa,n", [(1e2, 300), (1e3, 300), (1e4, 200), (1e3, 700)])
def test_fold_ill_conditioned_columns(hip, kappa, n):
    """Graded and correlated columns (X = U diag(s) V^T D with log-spaced s and a
    column scaling D over four decades): panels whose first CholeskyQR pass
    leaves the second-pass Gram far from the identity, or collapses, take the
    general Cholesky / inverse or the Householder fallback.  R^T R must stay
    within 4 kappa eps of X^T X."""
    rng = np.random.default_rng(int(kappa) + n)
    X = O.kappa_matrix(3 * n, n, kappa, rng) * np.logspace(0, -4, n)[rng.permutation(n)]
    Xt = torch.from_numpy(X).float().to(DEV)
    R, r = _fold_chunks(hip, [Xt], n)
    Ro = O.streaming_tsqr_update(None, Xt.double().cpu().numpy())
    assert r == n
    assert _gram_rel(R, Ro) <= 4 * _kappa(Ro) * EPS32


def test_fold_nan_gives_nonfinite_flag(hip):
    X = torch.randn(64, 16, device=DEV)
    X[3, 4] = float("nan")
    R, r = _fold_chunks(hip, [X], 16)
    Rd, flag = hip.finalize(R, 1 / 8.0, 1e-2, torch.float32, 0)
    assert flag.item() == 0
    X[3, 4] = 1.0
    R, r = _fold_chunks(hip, [X], 16)
    Rd, flag = hip.finalize(R, 1 / 8.0, 1e-2, torch.float32, 0)
    assert flag.item() == 1


def test_fold_is_deterministic(hip):
    X = torch.randn(3000, 700, device=DEV)
    R1, _ = _fold_chunks(hip, [X], 700, 1)
    R2, _ = _fold_chunks(hip, [X], 700, 1)
    assert torch.equal(R1, R2)


def test_fold_bf16_math_regression_bound(hip):
    g = torch.Generator(device=DEV).manual_seed(3)
    X = torch.randn(4096, 1024, device=DEV, generator=g)
    R, _ = _fold_chunks(hip, [X], 1024, 1)
    Ro = O.streaming_tsqr_update(None, X.double().cpu().numpy())
    e = _gram_rel(R, Ro)
    assert e <= 4 * _kappa(Ro) * EPS_BF16
    assert e < 2e-3   # measured regression bound for bf16 MFMA trailing updates


# --------------------------------------------------------------------------- finalize


@pytest.mark.parametrize("p,n,lam", [(500, 300, 1e-2), (4096, 1024, 1e-2), (64, 64, 1e-3),
                                      (3000, 1700, 1e-2)])
def test_finalize_matches_closed_form(hip, p, n, lam):
    g = torch.Generator(device=DEV).manual_seed(p + n)
    X = torch.randn(p, n, device=DEV, generator=g)
    R, r = _fold_chunks(hip, [X], n)
    Rd, flag = hip.finalize(R, 1 / math.sqrt(p), lam, torch.float32, 0)
    want = O.chol_factor([X.double().cpu().numpy()], p, lam)
    assert flag.item() == 1
    assert _gram_rel(Rd, want) <= 4 * _kappa(want) * EPS32
    Rb, _ = hip.finalize(R, 1 / math.sqrt(p), lam, torch.bfloat16, 0)
    assert torch.equal(Rb, Rd.to(torch.bfloat16))   # RNE cast of the same fp32 result


# --------------------------------------------------------------------------- fold + finalize


@pytest.mark.parametrize("prev,p,n,lam", [
    ([], 500, 300, 1e-2), ([300], 500, 300, 1e-2), ([64], 30, 128, 1e-2),
    ([], 64, 64, 1e-3), ([], 3000, 1700, 1e-2), ([1200], 1200, 2100, 1e-2), ([], 20, 50, 1e-1),
])
def test_fold_finalize_matches_closed_form(hip, prev, p, n, lam):
    """The fused call equals finalize(fold(R_in, X)): the R of [s R_in; s X; sqrt(lam) I]
    against the fp64 Cholesky closed form, and against the two-call path on the GPU."""
    g = torch.Generator(device=DEV).manual_seed(p + n + len(prev))
    Xs = [torch.randn(q, n, device=DEV, generator=g) for q in prev]
    X = torch.randn(p, n, device=DEV, generator=g)
    R, r = _fold_chunks(hip, Xs, n)
    R_before = R.clone()
    rows = sum(prev) + p
    Rd, flag = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.float32, 0)
    assert flag.item() == 1
    assert torch.equal(R, R_before)                  # the running factor is not touched
    want = O.chol_factor([x.double().cpu().numpy() for x in Xs + [X]], rows, lam)
    assert _gram_rel(Rd, want) <= 4 * _kappa(want) * EPS32
    Rg = Rd.double().cpu().numpy()
    assert np.all(np.diag(Rg) > 0) and not np.any(np.tril(Rg, -1))
    R2 = R.clone()
    r2 = hip.fold_(R2, r, X, 0)
    if r2 == n:
        Rd2, _ = hip.finalize(R2, 1 / math.sqrt(rows), lam, torch.float32, 0)
        assert _gram_rel(Rd, Rd2.double().cpu().numpy()) <= 4 * _kappa(want) * EPS32
    Rb, _ = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.bfloat16, 0)
    assert torch.equal(Rb, Rd.to(torch.bfloat16))   # RNE cast of the same fp32 result


def test_fold_finalize_guards_and_flags(hip):
    X = torch.randn(10, 20, device=DEV)
    with pytest.raises(Exception):
        hip.fold_finalize(None, 0, X, 1.0, 0.0, torch.float32, 0)   # 10 rows, 20 columns, no damping
    X = torch.randn(64, 16, device=DEV)
    X[3, 4] = float("nan")
    _, flag = hip.fold_finalize(None, 0, X, 1 / 8.0, 1e-2, torch.float32, 0)
    assert flag.item() == 0
    X[3, 4] = 1.0
    _, flag = hip.fold_finalize(None, 0, X, 1 / 8.0, 1e-2, torch.float32, 0)
    assert flag.item() == 1


# --------------------------------------------------------------------------- block CholeskyQR


@pytest.mark.parametrize("prev,p,n,lam", [
    ([], 500, 300, 1e-2), ([300], 500, 300, 1e-2), ([64], 30, 128, 1e-2),
    ([], 64, 64, 1e-3), ([], 3000, 1700, 1e-2), ([1200], 1200, 2100, 1e-2), ([], 20, 50, 1e-1),
    ([], 4000, 1536, 1e-2), ([], 1, 600, 1e-2), ([2000], 100, 1030, 1e-3),
])
def test_fold_finalize_cqr_matches_closed_form(hip, prev, p, n, lam):
    """Outer blocks factored by CholeskyQR2 + Householder reconstruction: the same
    R_damped as the panel path, within 4 kappa eps_fp32 of the fp64 Cholesky closed
    form, status 1, positive diagonal, exact zeros below it."""
    g = torch.Generator(device=DEV).manual_seed(p + n + len(prev))
    Xs = [torch.randn(q, n, device=DEV, generator=g) for q in prev]
    X = torch.randn(p, n, device=DEV, generator=g)
    R, r = _fold_chunks(hip, Xs, n)
    R_before = R.clone()
    rows = sum(prev) + p
    Rd, st = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.float32, 0, cqr=True)
    assert st.item() == 1
    assert torch.equal(R, R_before)
    want = O.chol_factor([x.double().cpu().numpy() for x in Xs + [X]], rows, lam)
    assert _gram_rel(Rd, want) <= 4 * _kappa(want) * EPS32
    Rg = Rd.double().cpu().numpy()
    assert np.all(np.diag(Rg) > 0) and not np.any(np.tril(Rg, -1))
    Rp, _ = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.float32, 0)
    assert _gram_rel(Rd, Rp.double().cpu().numpy()) <= 4 * _kappa(want) * EPS32
    Rb, st = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.bfloat16, 0, cqr=True)
    assert st.item() == 1 and torch.equal(Rb, Rd.to(torch.bfloat16))


@pytest.mark.parametrize("p,n,kappa", [(4096, 1024, 1e2), (6000, 2600, 1e1), (2048, 700, 1e2)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_fold_finalize_cqr_bf16_math(hip, p, n, kappa, xdt):
    """bf16 arithmetic against the fp64 closed form of the same (stored) input.  The
    block factorisation reads its columns as bf16, so an fp32 input carries the
    rounding of the data, 2^-9 relative per entry: a Gram error up to about
    2 * 2^-9 ~ 4e-3 (the panel path reads a block's own columns in fp32).  A bf16
    input is exact, and the result must then be as close as the panel path's."""
    rng = np.random.default_rng(p + n)
    X = torch.from_numpy(O.kappa_matrix(p, n, kappa, rng).astype(np.float32) * math.sqrt(p))
    X = X.to(xdt).to(DEV)
    lam = 1e-2
    want = O.chol_factor([X.double().cpu().numpy()], p, lam)
    Rd, st = hip.fold_finalize(None, 0, X, 1 / math.sqrt(p), lam, torch.float32, 1, cqr=True)
    assert st.item() == 1
    e = _gram_rel(Rd, want)
    Rp, _ = hip.fold_finalize(None, 0, X, 1 / math.sqrt(p), lam, torch.float32, 1)
    ep = _gram_rel(Rp, want)
    print(f"gram error cqr {e:.3e}, panels {ep:.3e}")
    assert e <= 4 * _kappa(want) * EPS_BF16
    if xdt == torch.float32:
        assert e < 4e-3
    else:
        assert e < 1.25 * ep + 1e-5


def test_fold_finalize_cqr_flags_ill_conditioned_blocks(hip):
    """A rank-deficient block (no damping, a zero column) and a non-finite input
    return status 2 (recompute with the panel path), which then gives the factor or
    the non-finite flag; a well-posed call after them is unaffected."""
    g = torch.Generator(device=DEV).manual_seed(5)
    X = torch.randn(900, 600, device=DEV, generator=g)
    X[:, 37] = 0.0
    _, st = hip.fold_finalize(None, 0, X, 1 / 30.0, 0.0, torch.float32, 0, cqr=True)
    assert st.item() == 2
    X2 = torch.randn(900, 600, device=DEV, generator=g)
    X2[:, 517] = 3.0 * X2[:, 12] - X2[:, 400]    # dependent columns across two blocks
    R2, st = hip.fold_finalize(None, 0, X2, 1 / 30.0, 0.0, torch.float32, 0, cqr=True)
    # the dependent column is rounding noise once the first block is applied:
    # either flagged, or factored with a backward error at fp32 level
    assert st.item() in (1, 2)
    if st.item() == 1:
        a = R2.double().cpu().numpy()
        x = X2.double().cpu().numpy() / 30.0
        assert np.linalg.norm(a.T @ a - x.T @ x) / np.linalg.norm(x.T @ x) < 1e-5
    X3 = torch.randn(900, 600, device=DEV, generator=g)
    X3[5, 5] = float("nan")
    _, st = hip.fold_finalize(None, 0, X3, 1 / 30.0, 1e-2, torch.float32, 0, cqr=True)
    assert st.item() == 2
    _, fl = hip.fold_finalize(None, 0, X3, 1 / 30.0, 1e-2, torch.float32, 0)
    assert fl.item() == 0
    X3[5, 5] = 0.5
    Rd, st = hip.fold_finalize(None, 0, X3, 1 / 30.0, 1e-2, torch.float32, 0, cqr=True)
    want = O.chol_factor([X3.double().cpu().numpy()], 900, 1e-2)
    assert st.item() == 1 and _gram_rel(Rd, want) <= 4 * _kappa(want) * EPS32


def test_fold_finalize_cqr_is_deterministic(hip):
    g = torch.Generator(device=DEV).manual_seed(11)
    X = torch.randn(3000, 1300, device=DEV, generator=g)
    for m in (0, 1):
        a, _ = hip.fold_finalize(None, 0, X, 1 / math.sqrt(3000), 1e-2, torch.float32, m, cqr=True)
        b, _ = hip.fold_finalize(None, 0, X, 1 / math.sqrt(3000), 1e-2, torch.float32, m, cqr=True)
        assert torch.equal(a, b)


@pytest.mark.parametrize("n_in,n_out,p", [(4096, 11008, 16384)])
def test_full_size_fold_finalize_bf16(hip, n_in, n_out, p):
    """The benchmarked factor update at full size in bf16 arithmetic, by the
    panel path and by CholeskyQR2 blocks: for 16 random probes v,
    ||R_d v||^2 = ||X v||^2 / p + lam ||v||^2 within 2e-3, and R_d upper
    triangular with a positive diagonal."""
    g = torch.Generator(device=DEV).manual_seed(7)
    for n, cqr in ((n_in, False), (n_out, False), (n_in, True), (n_out, True)):
        X = torch.randn(p, n, device=DEV, generator=g).to(torch.bfloat16)
        Rd, flag = hip.fold_finalize(None, 0, X, 1 / math.sqrt(p), 1e-2, torch.float32, 1, cqr=cqr)
        assert flag.item() == 1
        V = torch.randn(n, 16, device=DEV, generator=g, dtype=torch.float64)
        l2 = (Rd.double() @ V).norm(dim=0) ** 2
        r2 = (X.double() @ V).norm(dim=0) ** 2 / p + 1e-2 * (V ** 2).sum(0)
        assert ((l2 - r2).abs() / r2).max().item() < 2e-3
        d = torch.diagonal(Rd)
        assert bool((d > 0).all()) and torch.count_nonzero(torch.tril(Rd, -1)).item() == 0
        del X, Rd


# --------------------------------------------------------------------------- preconditioning


def _factors(p, n, lam, kappa, seed):
    rng = np.random.default_rng(seed)
    X = O.kappa_matrix(p, n, kappa, rng)
    return O.get_factor(O.streaming_tsqr_update(None, X), p, lam)


@pytest.mark.parametrize("n_out,n_in", [(32, 16), (256, 128), (1024, 1024), (300, 700), (10, 256)])
def test_precondition_fp32(hip, n_out, n_in):
    R_X = _factors(4 * n_in, n_in, 1e-2, 1e2, 1)
    R_G = _factors(4 * n_out, n_out, 1e-2, 1e1, 2)
    g = np.random.default_rng(3).normal(0, 0.1, (n_out, n_in))
    want = O.apply_vered(g, R_X, R_G)
    nat = hip.precondition(torch.tensor(g, dtype=torch.float32, device=DEV),
                           torch.tensor(R_X, dtype=torch.float32, device=DEV),
                           torch.tensor(R_G, dtype=torch.float32, device=DEV), 0)
    assert _rel(nat, want) <= 1e-5


@pytest.mark.parametrize("n_out,n_in", [(32, 16), (256, 128), (1024, 1024), (300, 700)])
def test_precondition_bf16(hip, n_out, n_in):
    R_X = O.bf16_round(_factors(4 * n_in, n_in, 1e-2, 1e2, 1).astype(np.float32))
    R_G = O.bf16_round(_factors(4 * n_out, n_out, 1e-2, 1e1, 2).astype(np.float32))
    g = np.random.default_rng(3).normal(0, 0.1, (n_out, n_in)).astype(np.float32)
    want = O.apply_vered(g.astype(np.float64), R_X.astype(np.float64), R_G.astype(np.float64))
    nat = hip.precondition(torch.tensor(g, device=DEV),
                           torch.tensor(R_X, device=DEV).to(torch.bfloat16),
                           torch.tensor(R_G, device=DEV).to(torch.bfloat16), 1)
    assert _rel(nat, want) <= 2e-2
    nat32 = hip.precondition(torch.tensor(g, device=DEV),
                             torch.tensor(R_X, device=DEV).to(torch.bfloat16),
                             torch.tensor(R_G, device=DEV).to(torch.bfloat16), 0)
    assert _rel(nat32, want) <= 1e-5     # fp32 arithmetic on bf16 factors: reference regime


def test_precondition_kappa_exposed(hip):
    """kappa(R_damped) ~ kappa(X) ~ 95: X scaled by sqrt(p), lambda below
    sigma_min^2 / 10.  The kernel gets the factors in fp32, and their rounding
    alone moves the four solves' result by up to kappa^2 eps32 (1e-3 here), for
    the reference as for this path; so the comparison is with fp64 solves on the
    same fp32 factors.  There the reference's own fp32 solves (four trsm,
    triangular.py:630-651, by LAPACK's strtrs) have their forward error, about
    kappa eps32 per solve; the HIP path (triangular inverses, then products)
    is held to 1e-5, or to twice the reference's error where that is larger."""
    n, p = 256, 1024
    rng = np.random.default_rng(7)
    X = O.kappa_matrix(p, n, 1e2, rng) * math.sqrt(p)
    R_X = O.get_factor(O.streaming_tsqr_update(None, X), p, 1e-5)
    kap = _kappa(R_X)
    assert kap > 50
    Rx32 = R_X.astype(np.float32)
    Rg32 = Rx32.copy()
    g32 = rng.normal(0, 0.1, (n, n)).astype(np.float32)
    exact = O.apply_vered(g32.astype(np.float64), Rx32.astype(np.float64),
                          Rg32.astype(np.float64))
    ref32 = O.apply_vered(g32, Rx32, Rg32)
    assert ref32.dtype == np.float32
    nat = hip.precondition(torch.tensor(g32, device=DEV), torch.tensor(Rx32, device=DEV),
                           torch.tensor(Rg32, device=DEV), 0)
    e, e_ref = _rel(nat, exact), _rel(ref32, exact)
    print(f"kappa {kap:.1f}: fp32 HIP {e:.2e}, reference fp32 solves {e_ref:.2e} "
          f"(against fp64 solves on the same fp32 factors)")
    assert e <= max(1e-5, 2 * e_ref)


def test_precondition_bias(hip):
    R_G = _factors(512, 128, 1e-2, 10.0, 5)
    g = np.random.default_rng(6).standard_normal(128)
    want = O.apply_vered_bias(g, R_G)
    Z = hip.tri_inverse(torch.tensor(R_G, dtype=torch.float32, device=DEV), 0)
    out = hip.precondition_bias(torch.tensor(g, dtype=torch.float32, device=DEV), Z)
    assert _rel(out, want) <= 1e-5


@pytest.mark.parametrize("n", [1, 63, 64, 65, 300, 1000, 2049])
def test_tri_inverse(hip, n):
    rng = np.random.default_rng(n)
    R = np.triu(rng.standard_normal((n, n))) / math.sqrt(n) + 2 * np.eye(n)
    Z = hip.tri_inverse(torch.tensor(R, dtype=torch.float32, device=DEV), 0)
    want = np.linalg.inv(R)
    assert _rel(Z, want) <= 1e-5
    assert np.all(np.tril(Z.cpu().numpy(), -1) == 0)


@pytest.mark.parametrize("n", [1, 63, 64, 65, 300, 1000, 2049])
def test_tri_inverse_bf16(hip, n):
    """bf16 factor and bf16 arithmetic (the transposed-copy doubling): Z against
    the fp64 inverse of the same bf16 matrix, at bf16 accuracy."""
    rng = np.random.default_rng(n + 7)
    R = np.triu(rng.standard_normal((n, n))) / math.sqrt(n) + 2 * np.eye(n)
    Rb = torch.tensor(R, dtype=torch.float32, device=DEV).to(torch.bfloat16)
    Z = hip.tri_inverse(Rb, 1)
    want = np.linalg.inv(Rb.double().cpu().numpy())
    assert _rel(Z, want) <= 2e-2
    assert np.all(np.tril(Z.cpu().numpy(), -1) == 0)


@pytest.mark.parametrize("n", [1, 65, 300, 2049])
def test_tri_inverse_bf16_copies(hip, n):
    """ifk_tri_inverse_bf16: the same Z as ifk_tri_inverse in bf16 arithmetic,
    bit for bit, and its bf16 copies are exactly the RNE roundings of Z and
    Z^T (other triangle zero)."""
    rng = np.random.default_rng(n + 11)
    R = np.triu(rng.standard_normal((n, n))) / math.sqrt(n) + 2 * np.eye(n)
    Rb = torch.tensor(R, dtype=torch.float32, device=DEV).to(torch.bfloat16)
    Z0 = hip.tri_inverse(Rb, 1)
    Z, Zb, ZT = hip.tri_inverse_bf16(Rb)
    assert torch.equal(Z, Z0)
    assert torch.equal(Zb, Z.bfloat16())
    assert torch.equal(ZT, Z.t().contiguous().bfloat16())


@pytest.mark.parametrize("n_out,n_in,trim", [(256, 128, False), (1100, 700, False),
                                             (300, 701, True)])
def test_precondition_apply_bf16_copies(hip, n_out, n_in, trim):
    """The apply from the bf16 copies equals the bf16 apply from fp32 Z bit for
    bit (it reads the same RNE values), also for the trimmed views IFKFAC
    passes with augment_bias."""
    R_X = O.bf16_round(_factors(4 * n_in, n_in, 1e-2, 1e2, 1).astype(np.float32))
    R_G = O.bf16_round(_factors(4 * n_out, n_out, 1e-2, 1e1, 2).astype(np.float32))
    RX = torch.tensor(R_X, device=DEV).to(torch.bfloat16)
    RG = torch.tensor(R_G, device=DEV).to(torch.bfloat16)
    ZX, ZXb, ZXt = hip.tri_inverse_bf16(RX)
    ZG, ZGb, ZGt = hip.tri_inverse_bf16(RG)
    m = n_in - 1 if trim else n_in
    if trim:
        ZX, ZXb, ZXt = ZX[:-1, :-1], ZXb[:-1, :-1], ZXt[:-1, :-1]
    g = torch.tensor(np.random.default_rng(3).normal(0, 0.1, (n_out, m)), dtype=torch.float32,
                     device=DEV)
    want = hip.precondition_apply(g, ZX.contiguous(), ZG, 1)
    got = hip.precondition_apply_bf16(g, (ZXb, ZXt), (ZGb, ZGt))
    assert torch.equal(got, want)
    if not trim:
        ref = O.apply_vered(g.double().cpu().numpy(), R_X.astype(np.float64),
                            R_G.astype(np.float64))
        assert _rel(got, ref) <= 2e-2


@pytest.mark.parametrize("n", [1, 65, 300, 2049])
def test_inverse_split_copies(hip, n):
    """ifk_inverse_split_copies: Z_hi = RNE(Z), Z_lo = RNE(Z - Z_hi) and the same
    halves of Z^T, exactly."""
    rng = np.random.default_rng(n + 13)
    R = np.triu(rng.standard_normal((n, n))) / math.sqrt(n) + 2 * np.eye(n)
    Z = hip.tri_inverse(torch.tensor(R, dtype=torch.float32, device=DEV), 0)
    hi, lo, thi, tlo = hip.inverse_split_copies(Z)
    assert torch.equal(hi, Z.bfloat16())
    assert torch.equal(lo, (Z - hi.float()).bfloat16())
    assert torch.equal(thi, hi.t().contiguous()) and torch.equal(tlo, lo.t().contiguous())


def _exposed_factor(p, n, kappa, seed):
    """kappa(R_damped) ~ kappa: X scaled by sqrt(p), lambda far below sigma_min^2."""
    rng = np.random.default_rng(seed)
    X = O.kappa_matrix(p, n, kappa, rng) * math.sqrt(p)
    return O.bf16_round(O.get_factor(O.streaming_tsqr_update(None, X), p, 1e-5).astype(np.float32))


@pytest.mark.parametrize("n_out,n_in,trim,exposed", [
    (256, 128, False, False), (1100, 700, False, False), (300, 701, True, False),
    (2100, 1500, False, False), (512, 256, False, True), (1300, 1024, False, True)])
def test_precondition_apply_x3(hip, n_out, n_in, trim, exposed):
    """The split-bf16 apply (three MFMA products per product from the hi/lo
    halves of the fp32 inverses) against fp64 solves on the same bf16 factors:
    within 4 * 2^-17 kappa(R_X) kappa(R_G), the accuracy of the split products
    through the kappa-amplifying solves, and far below the bf16 apply's error
    (a dropped lo half fails it); also for the trimmed views IFKFAC passes with
    augment_bias."""
    if exposed:
        R_X = _exposed_factor(4 * n_in, n_in, 1e2, 1)
        R_G = _exposed_factor(4 * n_out, n_out, 1e1, 2)
    else:
        R_X = O.bf16_round(_factors(4 * n_in, n_in, 1e-2, 1e2, 1).astype(np.float32))
        R_G = O.bf16_round(_factors(4 * n_out, n_out, 1e-2, 1e1, 2).astype(np.float32))
    RX = torch.tensor(R_X, device=DEV).to(torch.bfloat16)
    RG = torch.tensor(R_G, device=DEV).to(torch.bfloat16)
    ZX = hip.tri_inverse(RX, 0)
    ZG = hip.tri_inverse(RG, 0)
    sx, sg = hip.inverse_split_copies(ZX), hip.inverse_split_copies(ZG)
    m = n_in - 1 if trim else n_in
    if trim:
        sx = tuple(t[:-1, :-1] for t in sx)
    g = torch.tensor(np.random.default_rng(3).normal(0, 0.1, (n_out, m)), dtype=torch.float32,
                     device=DEV)
    got = hip.precondition_apply_x3(g, sx, sg)
    rx = R_X.astype(np.float64)[:m, :m] if trim else R_X.astype(np.float64)
    # trimming Z_X = R_X^{-1} to its leading block is the inverse of R_X's leading block
    ref = O.apply_vered(g.double().cpu().numpy(), rx, R_G.astype(np.float64))
    kx, kg = _kappa(rx), _kappa(R_G.astype(np.float64))
    e = _rel(got, ref)
    print(f"x3 apply {n_out}x{m}: rel {e:.3e}, kappa(R_X) {kx:.3g}, kappa(R_G) {kg:.3g}")
    assert e <= 4 * 2.0 ** -17 * kx * kg
    assert e <= 1e-3 * max(1.0, kx * kg / 100)
    if exposed:
        # the fp32-arithmetic apply on the same inverses, for scale
        e32 = _rel(hip.precondition_apply(g, ZX, ZG, 0), ref)
        print(f"  fp32 apply: rel {e32:.3e}")
    if not trim:
        ZXb, ZXt = sx[0], sx[2]
        eb = _rel(hip.precondition_apply_bf16(g, (ZXb, ZXt), (sg[0], sg[2])), ref)
        assert e <= eb / 10


@pytest.mark.parametrize("n,kappa", [(64, 1.0), (300, 3.0), (1100, 50.0), (2049, 1e3)])
@pytest.mark.parametrize("rdt", [torch.float32, torch.bfloat16])
def test_cond_estimate(hip, n, kappa, rdt):
    """ifk_cond_estimate against kappa_2(R) from the singular values (fp64, torch
    on the GPU as the checker): a lower bound within 10 % for factors of
    matrices with log-spaced singular values and a mean component, the
    inverse Z from the bf16-arithmetic triangular inverse IFKFAC uses.  The
    bound is 10 %: a factor's smallest singular values cluster when its input
    has a mean component, which slows the power iteration on Z."""
    rng = np.random.default_rng(n)
    X = O.kappa_matrix(4 * n, n, kappa, rng) + (0.5 if kappa > 1 else 0.0)
    R = O.get_factor(O.streaming_tsqr_update(None, X), 4 * n, 0.0 if kappa > 1 else 1.0)
    Rt = torch.tensor(R, dtype=torch.float32, device=DEV).to(rdt)
    Z = hip.tri_inverse_bf16(Rt)[0] if rdt == torch.bfloat16 else hip.tri_inverse(Rt, 0)
    got = hip.cond_estimate(Rt, Z).item()
    sv = torch.linalg.svdvals(Rt.double())
    want = (sv[0] / sv[-1]).item()
    assert got <= want * 1.001 + 1e-6
    assert got >= 0.9 * want


# --------------------------------------------------------------------------- update


@pytest.mark.parametrize("mom,wd,init", [(0.9, 0.0, True), (0.9, 0.01, False), (0.0, 0.1, False)])
def test_momentum_update(hip, mom, wd, init):
    rng = np.random.default_rng(8)
    W = rng.standard_normal((1000, 37)).astype(np.float32)
    nat = rng.standard_normal((1000, 37)).astype(np.float32)
    buf = rng.standard_normal((1000, 37)).astype(np.float32)
    Wt, bt, nt = (torch.tensor(a, device=DEV) for a in (W, buf, nat))
    hip.momentum_update_(nt, bt if mom > 0 else None, Wt, 0.05, mom, wd, init)
    Wo, bo = O.momentum_step(nat, None if init else buf, W, 0.05, mom, wd)
    assert np.allclose(Wt.cpu().numpy(), Wo, rtol=2e-7, atol=2e-7)
    if mom > 0:
        assert np.allclose(bt.cpu().numpy(), bo, rtol=2e-7, atol=2e-7)


# --------------------------------------------------------------------------- config: Linear 1024->1024


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_config_linear_1024_streaming_path(hip, mode):
    """8 chunks of X and delta (512 x 1024, stored bf16; kappa 1e2 / 1e1), damping 1e-2,
    gradient ~ N(0, 1e-2): fold, finalize, four solves; each stage against the oracle."""
    rng = np.random.default_rng(0)
    n, p, lam = 1024, 512, 1e-2
    Xs = [O.bf16_round(O.kappa_matrix(p, n, 1e2, rng).astype(np.float32)) for _ in range(8)]
    Ds = [O.bf16_round(O.kappa_matrix(p, n, 1e1, rng).astype(np.float32)) for _ in range(8)]
    grad = rng.normal(0, math.sqrt(1e-2), (n, n)).astype(np.float32)
    math_ = 0 if mode == "fp32" else 1
    RX = torch.zeros(n, n, device=DEV)
    RG = torch.zeros(n, n, device=DEV)
    rx = rg = 0
    RXo = RGo = None
    for X, D in zip(Xs, Ds):
        rx = hip.fold_(RX, rx, torch.tensor(X, device=DEV).to(torch.bfloat16), math_)
        rg = hip.fold_(RG, rg, torch.tensor(D, device=DEV).to(torch.bfloat16), math_)
        RXo = O.streaming_tsqr_update(RXo, X.astype(np.float64))
        RGo = O.streaming_tsqr_update(RGo, D.astype(np.float64))
        assert rx == RXo.shape[0] and rg == RGo.shape[0]
    tol_fold = 4 * _kappa(RXo) * (EPS32 if mode == "fp32" else EPS_BF16)
    assert _gram_rel(RX, RXo) <= tol_fold
    out_dt = torch.float32 if mode == "fp32" else torch.bfloat16
    FX, _ = hip.finalize(RX, 1 / math.sqrt(8 * p), lam, out_dt, math_)
    FG, _ = hip.finalize(RG, 1 / math.sqrt(8 * p), lam, out_dt, math_)
    FXo = O.get_factor(RXo, 8 * p, lam)
    FGo = O.get_factor(RGo, 8 * p, lam)
    st = EPS32 if mode == "fp32" else EPS_BF16
    assert _gram_rel(FX.float(), FXo) <= 4 * _kappa(FXo) * st
    nat = hip.precondition(torch.tensor(grad, device=DEV), FX, FG, math_)
    if mode == "fp32":
        want = O.apply_vered(grad.astype(np.float64), FXo, FGo)
        assert _rel(nat, want) <= 1e-5
    else:
        want = O.apply_vered(grad.astype(np.float64), O.bf16_round(FXo.astype(np.float32)).astype(np.float64),
                             O.bf16_round(FGo.astype(np.float32)).astype(np.float64))
        assert _rel(nat, want) <= 2e-2


# --------------------------------------------------------------------------- bf16_linalg


@pytest.mark.parametrize("n", [8, 32, 64, 256, 1000])
def test_bf16_qr_vs_cholesky_of_gram(hip, n):
    from ifkfac_amd import bf16_linalg as B
    g = torch.Generator(device=DEV).manual_seed(n)
    A = torch.randn(2 * n, n, device=DEV, generator=g).to(torch.bfloat16)
    R = B.block_householder_qr_bf16(A)
    assert R.dtype == torch.bfloat16 and R.shape == (n, n)
    Ad = A.double().cpu().numpy()
    want = np.linalg.cholesky(Ad.T @ Ad).T
    assert _rel(R, want) < 2e-2
    if n <= 32:   # the reference's own algorithm, restated
        Ro = O.positive_diagonal(O.householder_qr_bf16(Ad.astype(np.float32)).astype(np.float64))
        assert _rel(R, Ro) < 5e-2


@pytest.mark.parametrize("n", [8, 32, 64, 200])
def test_bf16_trsm_chol_inv(hip, n):
    from ifkfac_amd import bf16_linalg as B
    rng = np.random.default_rng(n)
    R = np.triu(rng.standard_normal((n, n))).astype(np.float32)
    R += np.diag(np.sign(np.diag(R)))
    Rb = O.bf16_round(R)
    Bm = O.bf16_round(rng.standard_normal((n, 4)).astype(np.float32))
    for upper in (True, False):
        T = Rb if upper else np.ascontiguousarray(Rb.T)
        X = B.solve_triangular_bf16(torch.tensor(T, device=DEV).bfloat16(),
                                    torch.tensor(Bm, device=DEV).bfloat16(), upper=upper)
        want = np.linalg.solve(T.astype(np.float64), Bm.astype(np.float64))
        assert _rel(X, want) < 5e-2
    Z = rng.standard_normal((2 * n, n)).astype(np.float32)
    S = O.bf16_round(Z.T @ Z + np.eye(n, dtype=np.float32))
    L = B.cholesky_bf16(torch.tensor(S, device=DEV).bfloat16()).double().cpu().numpy()
    assert np.linalg.norm(L @ L.T - S) / np.linalg.norm(S) < 2e-2
    assert np.all(np.triu(L, 1) == 0)
    Si = B.inv_spd_bf16(torch.tensor(S, device=DEV).bfloat16())
    assert _rel(Si, np.linalg.inv(S.astype(np.float64))) < 5e-2


def test_bf16_linalg_guards(hip):
    from ifkfac_amd import bf16_linalg as B
    with pytest.raises(TypeError):
        B.solve_triangular_bf16(torch.eye(4, device=DEV), torch.ones(4, 1, device=DEV).bfloat16())
    with pytest.raises(ValueError):
        B.solve_triangular_bf16(torch.ones(4, 3, device=DEV).bfloat16(),
                                torch.ones(4, 1, device=DEV).bfloat16())
    with pytest.raises(AssertionError):
        B.block_householder_qr_bf16(torch.randn(3, 5, device=DEV).bfloat16())


@pytest.mark.parametrize("n", [8, 100])
@pytest.mark.parametrize("upper", [True, False])
@pytest.mark.parametrize("dv", [5e-8, -5e-8, 0.0, -0.0])
def test_bf16_trsm_tiny_and_zero_diagonals(hip, n, upper, dv):
    """solve_triangular_bf16 through the _safe_div clamp (bf16_linalg.py:44-59,
    :233/:241): a diagonal entry below 1e-7 in magnitude divides by
    sign(d) 1e-7, with sign(0) = +1 for 0 and -0.0.  One clamped pivot per
    matrix (two make the solve too ill-conditioned for a forward error to
    mean anything).  Against the oracle's substitution and against the fp64
    solve with the clamped diagonal, at the bf16 bound of the general solve
    test; n = 100 crosses the 64-block doubling of the inverse."""
    from ifkfac_amd import bf16_linalg as B
    rng = np.random.default_rng(n + (0 if upper else 1))
    R = np.triu(rng.standard_normal((n, n)) * 0.1).astype(np.float32)
    d = rng.choice([2.0, -1.5, 1.0, 3.0], n).astype(np.float32)
    d[n // 2] = dv
    np.fill_diagonal(R, d)
    R = O.bf16_round(R)
    if not upper:
        R = np.ascontiguousarray(R.T)
    Bm = O.bf16_round(rng.standard_normal((n, 3)).astype(np.float32))
    X = B.solve_triangular_bf16(torch.tensor(R, device=DEV).bfloat16(),
                                torch.tensor(Bm, device=DEV).bfloat16(), upper=upper)
    Xo = O.solve_triangular_bf16(R, Bm, upper=upper)
    Rc = R.astype(np.float64)
    Rc[n // 2, n // 2] = -1e-7 if dv < 0 else 1e-7       # -0.0 < 0 is False: +1e-7
    Xt = np.linalg.solve(Rc, Bm.astype(np.float64))
    assert bool(torch.isfinite(X).all())
    assert _rel(X, Xt) < 2e-2
    assert _rel(X, Xo.astype(np.float64)) < 2e-2
    # the clamped row carries the divisor's sign (1e7 scale): signs as the oracle's
    Xg = X.double().cpu().numpy()
    assert np.array_equal(np.sign(Xg[n // 2]), np.sign(Xo[n // 2].astype(np.float64)))
    assert np.abs(Xg[n // 2]).max() > 1e5


def test_bf16_cholesky_pivot_clamp_cases(hip):
    """cholesky_bf16's pivot rule (bf16_linalg.py:258-260) on the oracle's hand
    cases: singular (rank 1) and indefinite inputs clamp at 1e-7 and match the
    oracle bit for bit; a NaN pivot propagates (clamp_min keeps NaN); a larger
    block-diagonal input with a rank-deficient part (n = 100, two 64-blocks)
    matches it to the bf16 bound."""
    from ifkfac_amd import bf16_linalg as B
    u = np.array([1.0, 2.0, -3.0, 1.0], np.float32)
    cases = [np.outer(u, u),
             np.array([[4.0, 2.0, 0.0], [2.0, -3.0, 0.0], [0.0, 0.0, 9.0]], np.float32),
             np.ones((40, 40), np.float32)]
    for A in cases:
        L = B.cholesky_bf16(torch.tensor(A, device=DEV).bfloat16()).float().cpu().numpy()
        assert np.array_equal(L, O.cholesky_bf16(A)), A.shape
    A = np.eye(8, dtype=np.float32)
    A[0, 0] = np.nan
    L = B.cholesky_bf16(torch.tensor(A, device=DEV).bfloat16()).float().cpu().numpy()
    assert np.isnan(L[np.tril_indices(8)]).all() and not np.any(np.triu(L, 1))
    rng = np.random.default_rng(9)
    n, k = 100, 40
    A = np.zeros((n, n), np.float32)
    v = rng.integers(-2, 3, k).astype(np.float32)
    v[0] = 1.0
    A[:k, :k] = np.outer(v, v)                      # rank 1: clamped pivots
    Z = rng.standard_normal((2 * (n - k), n - k)).astype(np.float32)
    A[k:, k:] = O.bf16_round(Z.T @ Z / (n - k) + np.eye(n - k, dtype=np.float32))
    L = B.cholesky_bf16(torch.tensor(A, device=DEV).bfloat16()).float().cpu().numpy()
    Lo = O.cholesky_bf16(A)
    assert np.all(np.isfinite(L))
    assert np.linalg.norm(L - Lo) / np.linalg.norm(Lo) < 2e-2
    r = float(O.bf16_round(np.array([math.sqrt(1e-7)], np.float32))[0])
    assert np.array_equal(np.diag(L)[1:k], np.full(k - 1, r, np.float32))


# --------------------------------------------------------------------------- full sizes


@pytest.mark.parametrize("p,n,dt", [(16384, 4096, torch.bfloat16), (16384, 11008, torch.bfloat16),
                                    (8192, 4096, torch.float32)])
def test_full_size_fold_properties(hip, p, n, dt):
    """At full layer sizes: for random probes v, ||R v|| = ||X v|| (R^T R = X^T X),
    R upper triangular with positive diagonal, finalize gives R_d^T R_d = R^T R/p + lam I."""
    g = torch.Generator(device=DEV).manual_seed(n)
    X = torch.randn(p, n, device=DEV, generator=g).to(dt)
    R = torch.zeros(n, n, device=DEV)
    r = hip.fold_(R, 0, X, 1 if dt == torch.bfloat16 else 0)
    assert r == n
    V = torch.randn(n, 16, device=DEV, generator=g, dtype=torch.float64)
    lhs = (R.double() @ V).norm(dim=0)
    rhs = (X.double() @ V).norm(dim=0)
    tol = 2e-3 if dt == torch.bfloat16 else 1e-5
    assert ((lhs - rhs).abs() / rhs).max().item() < tol
    d = torch.diagonal(R)
    assert bool((d > 0).all())
    assert torch.count_nonzero(torch.tril(R, -1)).item() == 0
    Rd, flag = hip.finalize(R, 1 / math.sqrt(p), 1e-2, torch.float32,
                            1 if dt == torch.bfloat16 else 0)
    assert flag.item() == 1
    l2 = (Rd.double() @ V).norm(dim=0) ** 2
    r2 = (R.double() @ V).norm(dim=0) ** 2 / p + 1e-2 * (V ** 2).sum(0)
    assert ((l2 - r2).abs() / r2).max().item() < tol


def test_full_size_precondition_residual(hip):
    """4096 -> 11008 layer: R_G^T R_G nat R_X^T R_X reproduces grad.  The factors are
    damped factors of random data with p = 2n rows, so kappa(A) = kappa(R)^2 <= 30
    (Marchenko-Pastur edges (1 -+ 1/sqrt(2))^2 plus damping).  A backward-stable
    solve leaves a residual of order kappa(A) kappa(G) eps_fp32 ~ 1e-4 in fp32
    arithmetic; bf16 arithmetic is held to the 2e-2 natural-gradient bound."""
    n_in, n_out = 4096, 11008
    g = torch.Generator(device=DEV).manual_seed(0)

    def factor(n):
        X = torch.randn(2 * n, n, device=DEV, generator=g)
        R = torch.zeros(n, n, device=DEV)
        hip.fold_(R, 0, X, 0)
        Rd, _ = hip.finalize(R, 1 / math.sqrt(2 * n), 1e-2, torch.float32, 0)
        return Rd

    RX, RG = factor(n_in), factor(n_out)
    grad = torch.randn(n_out, n_in, device=DEV, generator=g) * 0.1
    for math_, dt, tol in ((0, torch.float32, 1e-4), (1, torch.bfloat16, 2e-2)):
        rx, rg = RX.to(dt), RG.to(dt)
        nat = hip.precondition(grad, rx, rg, math_)
        rxd, rgd = rx.double(), rg.double()
        back = rgd.t() @ (rgd @ nat.double() @ rxd.t()) @ rxd
        assert ((back - grad.double()).norm() / grad.double().norm()).item() < tol


@pytest.mark.parametrize("n", [300, 700, 3000, 4096])
@pytest.mark.parametrize("rdt", [torch.float32, torch.bfloat16])
def test_tri_inverse_x3(hip, n, rdt):
    """ifk_tri_inverse_x3 against the fp64 inverse of the same (fp32 or
    bf16-valued) factor: the split levels (512 wide and up; ragged pairs at
    700 and 3000, none at 300) keep the error within 8 kappa 2^-17 and within
    four times the fp32-arithmetic inverse's own error plus 2^-17."""
    g = torch.Generator(device=DEV).manual_seed(n)
    X = torch.randn(2 * n, n, device=DEV, generator=g, dtype=torch.float64)
    X[:, : n // 3] *= 10.0
    R = torch.linalg.qr(X, mode="r")[1]
    R = R * torch.sign(torch.diagonal(R)).unsqueeze(1)
    Rt = R.to(rdt)
    R64 = Rt.double()
    Z64 = torch.linalg.inv(R64)
    kap = float(torch.linalg.cond(R64))
    Zx = hip.tri_inverse_x3(Rt).double()
    Zf = hip.tri_inverse(Rt, 0).double()
    ex = float((Zx - Z64).norm() / Z64.norm())
    ef = float((Zf - Z64).norm() / Z64.norm())
    print(f"n {n} {rdt}: kappa {kap:.1f}, x3 {ex:.2e}, fp32 {ef:.2e}")
    assert ex <= 8 * kap * 2.0 ** -17
    assert ex <= 4 * ef + 2.0 ** -17
    assert bool(torch.isfinite(Zx).all()) and float(torch.tril(Zx, -1).abs().max()) == 0.0


def test_triangular_mirrors_on_gpu(hip):
    """The function-level mirrors of ifkfac/triangular.py on the GPU against the
    oracle: streaming update (trapezoid, then square), tsqr, the bucket fold,
    finalize_R, apply_vered (fp32 and bf16 factors), apply_vered_batched and
    apply_vered_bias (two triangular solves)."""
    from ifkfac_amd import triangular as T
    rng = np.random.default_rng(33)
    X1, X2 = rng.standard_normal((100, 300)), rng.standard_normal((700, 300))
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    R = T.streaming_tsqr_update(T.streaming_tsqr_update(None, t(X1)), t(X2))
    want = O.streaming_tsqr_update(O.streaming_tsqr_update(None, X1), X2)
    assert _gram_rel(R.double().cpu().numpy(), want) <= 4 * _kappa(want) * EPS32
    Rt = T.tsqr(t(X2)).double().cpu().numpy()
    assert _gram_rel(Rt, O.streaming_tsqr_update(None, X2)) <= 1e-5
    Rb = T.batched_streaming_tsqr_update(torch.zeros(2, 300, 300, device=DEV),
                                         t(np.stack([X2, 0.5 * X2])))
    assert _gram_rel(Rb[1].double().cpu().numpy(),
                        O.streaming_tsqr_update(None, 0.5 * X2)) <= 1e-5
    Rd = T.finalize_R(t(want), 1e-2).double().cpu().numpy()
    assert np.linalg.norm(Rd.T @ Rd - want.T @ want - 1e-2 * np.eye(300)) <= \
        1e-5 * np.linalg.norm(want.T @ want)
    R_X = O.get_factor(O.streaming_tsqr_update(None, X2), 700, 1e-2)
    R_G = O.get_factor(O.streaming_tsqr_update(None, rng.standard_normal((900, 200))), 900, 1e-2)
    g = rng.standard_normal((200, 300))
    ref = O.apply_vered(g, R_X, R_G)
    assert _rel(T.apply_vered(t(g), t(R_X), t(R_G)), ref) <= 1e-5
    Rxb, Rgb = O.bf16_round(R_X.astype(np.float32)), O.bf16_round(R_G.astype(np.float32))
    nat_b = T.apply_vered(t(g), t(Rxb).bfloat16(), t(Rgb).bfloat16())
    assert _rel(nat_b, O.apply_vered(g, Rxb.astype(np.float64), Rgb.astype(np.float64))) <= 2e-2
    natb = T.apply_vered_batched(t(np.stack([g, 2 * g])), t(np.stack([R_X, R_X])),
                                 t(np.stack([R_G, R_G])))
    assert _rel(natb[1], 2 * ref) <= 1e-5
    gb = rng.standard_normal(200)
    assert _rel(T.apply_vered_bias(t(gb), t(R_G)), O.apply_vered_bias(gb, R_G)) <= 1e-5


def test_triangular_api_helpers_on_gpu(hip):
    """The reference module's off-path helpers (triangular.py:89-143, 150-227,
    331-379, 506-544) on the GPU: tsqr honours tile_size (700 rows in tiles of
    128: the same R as one fold, against the oracle); sgso's Q has orthonormal
    columns and Q R = M, R the oracle's; the bucket fold in bf16 arithmetic
    takes one batched Gram-route fold (each entry's factor that of its
    bf16-rounded rows within 1e-4) and folds an entry the Gram route
    refuses -- a repeated column at 1e3 times the others' scale -- by the
    panel path; apply_vered_batched with bf16 factors runs the batched apply,
    each entry bit for bit tri_inverse_bf16 + precondition_apply_bf16, within
    2e-2 of fp64 solves on the same factors."""
    from ifkfac_amd import triangular as T
    from ifkfac_amd._backend import MATH_BF16
    rng = np.random.default_rng(34)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    X = rng.standard_normal((700, 300))
    want = O.streaming_tsqr_update(None, X)
    Rt = T.tsqr(t(X), tile_size=128).double().cpu().numpy()
    assert _gram_rel(Rt, want) <= 1e-5
    with pytest.raises(ValueError):
        T.tsqr(t(X), tile_size=0)
    Q, R = T.sgso(t(X))
    Qd, Rd = Q.double().cpu().numpy(), R.double().cpu().numpy()
    assert _gram_rel(Rd, want) <= 1e-5 and bool((np.diag(Rd) > 0).all())
    assert np.linalg.norm(Qd.T @ Qd - np.eye(300)) <= 1e-4 * np.sqrt(300)
    assert np.linalg.norm(Qd @ Rd - X) <= 1e-5 * np.linalg.norm(X)
    with pytest.raises(ValueError):
        T.sgso(t(X[:100]))
    # bucket fold, bf16 arithmetic: entries 0 and 2 by the Gram route, entry 1 refused
    n, p = 256, 1024
    R0 = torch.stack([t(O.streaming_tsqr_update(None, rng.standard_normal((p, n))))
                      for _ in range(3)])
    chunks = np.stack([rng.standard_normal((p, n)) for _ in range(3)])
    chunks[1][:, 5] *= 1e3
    chunks[1][:, 9] = chunks[1][:, 5]
    calls = [0]
    real = type(hip).fold_gram_batched_

    def wrap(self, *a):
        calls[0] += 1
        return real(self, *a)

    type(hip).fold_gram_batched_ = wrap
    try:
        Rb = T.batched_streaming_tsqr_update(R0, t(chunks), math=MATH_BF16)
    finally:
        type(hip).fold_gram_batched_ = real
    assert calls[0] == 1
    for i in range(3):
        r0 = R0[i].double().cpu().numpy()
        rows = O.bf16_round(chunks[i].astype(np.float32)).astype(np.float64)
        got = Rb[i].double().cpu().numpy()
        if i == 1:
            # the panel path in fp32 arithmetic on the rows as given
            ref_i = O.streaming_tsqr_update(r0, chunks[i])
            assert _gram_rel(got, ref_i) <= 4 * _kappa(ref_i) * EPS32
        else:
            # the chunk's rows as bf16 (their RNE rounding), the running
            # factor split hi + lo (fp32 to about 2^-16)
            ref_i = O.streaming_tsqr_update(r0, rows)
            assert _gram_rel(got, ref_i) <= 1e-4, i
    # bucket apply, bf16 factors
    R_X = O.get_factor(O.streaming_tsqr_update(None, rng.standard_normal((900, 256))), 900, 1e-2)
    R_G = O.get_factor(O.streaming_tsqr_update(None, rng.standard_normal((900, 192))), 900, 1e-2)
    Rxb = torch.stack([t(R_X), t(2 * R_X)]).bfloat16()
    Rgb = torch.stack([t(R_G), t(R_G)]).bfloat16()
    G = t(rng.standard_normal((2, 192, 256)))
    natb = T.apply_vered_batched(G, Rxb, Rgb)
    for i in range(2):
        _, zxb, zxt = hip.tri_inverse_bf16(Rxb[i])
        _, zgb, zgt = hip.tri_inverse_bf16(Rgb[i])
        one = hip.precondition_apply_bf16(G[i], (zxb, zxt), (zgb, zgt))
        assert torch.equal(natb[i], one), i
        ref = O.apply_vered(G[i].double().cpu().numpy(), Rxb[i].double().cpu().numpy(),
                            Rgb[i].double().cpu().numpy())
        assert _rel(natb[i], ref) <= 2e-2
