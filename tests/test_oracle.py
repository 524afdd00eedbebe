"""Pins the CPU oracle (oracle/ifk_oracle.py) before anything is checked against it.

Each oracle function is checked against what the mathematics fixes (closed
forms, uniqueness of the positive-diagonal R factor, exact rational
arithmetic on tiny inputs, hand-computed rounding cases) and against the
recipe tests the reference itself ships (tests/test_equivalence.py,
tests/test_bf16_stability.py of the reference, restated on the oracle).
A few tests plant a plausible mistake in a copy of an oracle function and
assert that the same check rejects it, so the checks are shown to bite.
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ifk_oracle as O

# --------------------------------------------------------------------------- bf16


def test_bf16_round_hand_cases():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)       # bf16 spacing at 1.0
    half = np.float32(2.0 ** -8)
    cases = {
        1.0: 1.0,
        float(one + half): 1.0,                      # tie -> even (mantissa 0)
        float(one + ulp + half): float(one + 2 * ulp),  # tie -> even (mantissa 2)
        float(one + half + np.float32(2.0 ** -20)): float(one + ulp),  # above the tie
        -0.0: -0.0,
        float("inf"): float("inf"),
        3.4028234663852886e38: float("inf"),         # max fp32 rounds up past bf16 max
        3.3895313892515355e38: 3.3895313892515355e38,  # bf16 max is exact
    }
    for x, want in cases.items():
        got = float(O.bf16_round(np.array([x], np.float32))[0])
        assert got == want or (math.isnan(got) and math.isnan(want)), (x, got, want)
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32))[0])
    assert np.signbit(O.bf16_round(np.array([-0.0], np.float32))[0])


def test_bf16_round_matches_torch_bitwise():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * (10.0 ** rng.integers(-30, 30, 100000)),
                        np.array([1e-40, -1e-41, 6e-39], np.float32)]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = O.bf16_round(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# --------------------------------------------------------------------------- R factors


def test_positive_diagonal_hand_case():
    R = np.array([[-2.0, 1.0, 3.0], [0.0, 0.0, -5.0], [0.0, 0.0, -1.0]])
    want = np.array([[2.0, -1.0, -3.0], [0.0, 0.0, -5.0], [0.0, 0.0, 1.0]])
    assert np.array_equal(O.positive_diagonal(R), want)


def test_gram_pivot_ratio_closed_forms():
    """Two unit columns at angle t: ratios (1, sin^2 t); orthogonal columns of any
    length: all 1; a repeated column: 0.  A planted variant that divides by the
    pivot's own column norm after the update (always 1) fails the angle case."""
    for t in (0.7, 1e-2, 1e-3):
        P = np.array([[1.0, math.cos(t)], [0.0, math.sin(t)], [0.0, 0.0]])
        r = O.gram_pivot_ratio(P)
        assert abs(r[0] - 1.0) < 1e-15 and abs(r[1] - math.sin(t) ** 2) <= 1e-12 * math.sin(t) ** 2
        planted = np.diag(np.linalg.qr(P, mode="r")) ** 2 / np.diag(np.linalg.qr(P, mode="r")) ** 2
        assert abs(planted[1] - math.sin(t) ** 2) > 1e-3
    Q = np.linalg.qr(np.random.default_rng(0).standard_normal((9, 4)))[0] * np.array([3, .1, 7, 1])
    assert np.allclose(O.gram_pivot_ratio(Q), 1.0, rtol=1e-12)
    P = np.random.default_rng(1).standard_normal((6, 3))
    P[:, 2] = P[:, 0]
    assert O.gram_pivot_ratio(P)[2] < 1e-25


def _gs_exact(A):
    """R of Gram-Schmidt in exact rationals, returned as R^T R (sqrt-free form):
    the Gram matrix A^T A itself, built from Fractions."""
    m, n = len(A), len(A[0])
    return [[sum(Fraction(A[k][i]) * Fraction(A[k][j]) for k in range(m)) for j in range(n)]
            for i in range(n)]


def test_fold_tiny_integer_exact_gram():
    A = [[1, 2, 0], [3, -1, 4], [0, 5, 1], [2, 2, -3], [1, 0, 0]]
    X = np.array(A, dtype=np.float64)
    R = O.streaming_tsqr_update(O.streaming_tsqr_update(None, X[:2]), X[2:])
    G = _gs_exact(A)
    RtR = R.T @ R
    for i in range(3):
        for j in range(3):
            assert abs(RtR[i, j] - float(G[i][j])) < 1e-12
    assert np.all(np.diag(R) > 0)
    assert np.allclose(np.tril(R, -1), 0)


@pytest.mark.parametrize("chunks,n", [([64, 64], 40), ([30, 30, 100], 50), ([5, 7, 3], 20),
                                      ([512] * 3, 96)])
def test_fold_equals_cholesky_of_gram(chunks, n):
    rng = np.random.default_rng(1)
    R = None
    Xs = []
    for p in chunks:
        X = rng.standard_normal((p, n))
        Xs.append(X)
        R = O.streaming_tsqr_update(R, X)
        rows = sum(x.shape[0] for x in Xs)
        assert R.shape == (min(rows, n), n)
        if rows >= n:
            want = O.chol_factor(Xs, 1, 0.0)
            assert np.abs(R - want).max() < 1e-10 * np.abs(want).max()


def test_fold_check_rejects_planted_mistakes():
    rng = np.random.default_rng(2)
    X1, X2 = rng.standard_normal((50, 20)), rng.standard_normal((50, 20))
    want = O.chol_factor([X1, X2], 1, 0.0)

    def no_sign(Rold, X):  # forgets the positive-diagonal normalisation
        Rn = np.linalg.qr(X, mode="r")
        return Rn if Rold is None else np.linalg.qr(np.vstack([Rold, Rn]), mode="r")

    def drops_old(Rold, X):  # merges without the running factor
        return O.positive_diagonal(np.linalg.qr(X, mode="r"))

    for bad in (no_sign, drops_old):
        R = bad(bad(None, X1), X2)
        assert np.abs(R - want).max() > 1e-3


def test_finalize_and_get_factor_closed_form():
    rng = np.random.default_rng(3)
    Xs = [rng.standard_normal((100, 30)) for _ in range(3)]
    R = None
    for X in Xs:
        R = O.streaming_tsqr_update(R, X)
    lam = 1e-2
    got = O.get_factor(R, 300, lam)
    want = O.chol_factor(Xs, 300, lam)
    assert np.abs(got - want).max() < 1e-12
    # the check fails for a plausible mistake: damping added as lambda^2
    bad = O.positive_diagonal(np.linalg.qr(np.vstack([R / math.sqrt(300), lam * np.eye(30)]),
                                           mode="r"))
    assert np.abs(bad - want).max() > 1e-4
    assert O.get_factor(R[:20], 300, lam) is None       # non-square: skipped
    assert O.get_factor(None, 0, lam) is None


# --------------------------------------------------------------------------- solves


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_apply_vered_matches_classic_fp64(seed):
    """Restates the reference's test_ifkfac_matches_classic_fp64 on the oracle."""
    rng = np.random.default_rng(seed)
    p, n_in, n_out, lam = 128, 16, 32, 1e-2
    X = rng.standard_normal((p, n_in))
    dY = rng.standard_normal((p, n_out))
    g = rng.standard_normal((n_out, n_in))
    R_X = O.get_factor(O.streaming_tsqr_update(None, X), p, lam)
    R_G = O.get_factor(O.streaming_tsqr_update(None, dY), p, lam)
    got = O.apply_vered(g, R_X, R_G)
    want = O.natgrad_closed_form(X, dY, g, lam)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-10
    # planted mistakes: swapped factor sides, or one transpose dropped
    bad1 = O.apply_vered(g.T, R_G, R_X).T if n_in == n_out else None
    bad2 = np.linalg.solve(R_G.T, g) @ np.linalg.inv(R_X.T @ R_X)
    assert np.linalg.norm(bad2 - want) / np.linalg.norm(want) > 1e-2
    del bad1


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_apply_vered_fp32_recipe(seed):
    rng = np.random.default_rng(seed)
    p, n_in, n_out, lam = 256, 16, 32, 1e-2
    X = rng.standard_normal((p, n_in)).astype(np.float32)
    dY = rng.standard_normal((p, n_out)).astype(np.float32)
    g = rng.standard_normal((n_out, n_in)).astype(np.float32)
    R_X = O.get_factor(O.streaming_tsqr_update(None, X), p, lam).astype(np.float32)
    R_G = O.get_factor(O.streaming_tsqr_update(None, dY), p, lam).astype(np.float32)
    got = O.apply_vered(g, R_X, R_G)
    want = O.natgrad_closed_form(X.astype(np.float64), dY.astype(np.float64), g.astype(np.float64), lam)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-3


def test_bf16_kappa_contrast():
    """Restates the reference's test_ifkfac_beats_classic_at_bf16_high_kappa."""
    rng = np.random.default_rng(0)
    p, n, kappa, lam = 1024, 16, 100.0, 1e-3
    U = O.haar(p, n, rng)
    V = O.haar(n, n, rng)
    s = np.logspace(0, math.log10(kappa), n)
    X = (U * s) @ V.T
    dY = rng.standard_normal((p, n))
    g = rng.standard_normal((n, n))
    ref = O.natgrad_closed_form(X, dY, g, lam)
    A = O.bf16_round((X.T @ X / p).astype(np.float32)).astype(np.float64)
    G = O.bf16_round((dY.T @ dY / p).astype(np.float32)).astype(np.float64)
    classic = np.linalg.solve(G + lam * np.eye(n), g) @ np.linalg.inv(A + lam * np.eye(n))
    Xb = O.bf16_round(X.astype(np.float32)).astype(np.float64)
    Db = O.bf16_round(dY.astype(np.float32)).astype(np.float64)
    R_X = O.bf16_round(O.get_factor(O.streaming_tsqr_update(None, Xb), p, lam).astype(np.float32))
    R_G = O.bf16_round(O.get_factor(O.streaming_tsqr_update(None, Db), p, lam).astype(np.float32))
    ifk = O.apply_vered(g, R_X.astype(np.float64), R_G.astype(np.float64))
    e_c = np.linalg.norm(classic - ref) / np.linalg.norm(ref)
    e_i = np.linalg.norm(ifk - ref) / np.linalg.norm(ref)
    assert e_c > 5 * e_i


def test_apply_vered_bias_closed_form():
    rng = np.random.default_rng(4)
    D = rng.standard_normal((200, 12))
    lam = 1e-2
    R_G = O.get_factor(O.streaming_tsqr_update(None, D), 200, lam)
    g = rng.standard_normal(12)
    want = np.linalg.solve(D.T @ D / 200 + lam * np.eye(12), g)
    assert np.abs(O.apply_vered_bias(g, R_G) - want).max() < 1e-10


# --------------------------------------------------------------------------- update rules


def test_momentum_step_unrolled():
    W0 = np.array([1.0, -2.0, 0.5], np.float32)
    n1 = np.array([0.1, 0.2, -0.3], np.float32)
    n2 = np.array([-0.5, 0.0, 1.0], np.float32)
    lr, mu, wd = 0.1, 0.9, 0.01
    W1, b1 = O.momentum_step(n1, None, W0, lr, mu, wd)
    W2, b2 = O.momentum_step(n2, b1, W1, lr, mu, wd)
    # by hand: b1 = n1; W1 = W0 (1 - lr wd) - lr b1; b2 = mu b1 + n2; W2 = W1 (1 - lr wd) - lr b2
    assert np.allclose(b1, n1, atol=0)
    assert np.allclose(W1, W0 * (1 - lr * wd) - lr * n1, rtol=1e-6)
    assert np.allclose(b2, mu * n1 + n2, rtol=1e-6)
    assert np.allclose(W2, W1 * (1 - lr * wd) - lr * (mu * n1 + n2), rtol=1e-6)
    # no momentum: plain SGD, no buffer
    W, b = O.momentum_step(n1, None, W0, lr, 0.0, 0.0)
    assert b is None and np.allclose(W, W0 - lr * n1, rtol=1e-7)


def test_schedule():
    assert all(O.should_update_factors(s, 1) for s in range(1, 30))
    hits = [s for s in range(1, 41) if O.should_update_factors(s, 10)]
    assert hits == [10, 20, 30, 40]


# --------------------------------------------------------------------------- bf16_linalg


@pytest.mark.parametrize("n", [8, 16])
def test_bf16_linalg_restatements_tolerance(n):
    rng = np.random.default_rng(5)
    A = rng.standard_normal((2 * n, n)).astype(np.float32)
    R = O.householder_qr_bf16(A)
    Rt = np.linalg.cholesky(A.astype(np.float64).T @ A.astype(np.float64)).T
    Rn = O.positive_diagonal(R.astype(np.float64))
    assert np.linalg.norm(Rn - Rt) / np.linalg.norm(Rt) < 5e-2
    S = A.T @ A + np.eye(n, dtype=np.float32)
    L = O.cholesky_bf16(S)
    assert np.linalg.norm(L @ L.T - S) / np.linalg.norm(S) < 5e-2
    Rtri = np.triu(rng.standard_normal((n, n))).astype(np.float32)
    Rtri += np.diag(np.sign(np.diag(Rtri)))
    B = rng.standard_normal((n, 3)).astype(np.float32)
    X = O.solve_triangular_bf16(Rtri, B, upper=True)
    Xt = np.linalg.solve(Rtri.astype(np.float64), B)
    assert np.linalg.norm(X - Xt) / np.linalg.norm(Xt) < 1e-1
    Ai = O.inv_spd_bf16(S)
    St = np.linalg.inv(S.astype(np.float64))
    assert np.linalg.norm(Ai - St) / np.linalg.norm(St) < 1e-1


def test_kappa_matrix_condition():
    rng = np.random.default_rng(6)
    X = O.kappa_matrix(512, 256, 100.0, rng)
    s = np.linalg.svd(X, compute_uv=False)
    assert abs(s[0] - 1.0) < 1e-10 and abs(s[-1] - 0.01) < 1e-12


# --------------------------------------------------------------------------- bf16_linalg special cases
#
# The clamps and skips of bf16_linalg.py (_safe_div :44-59, cholesky_bf16's
# clamp_min(1e-7) pivot :258-260, the zero-norm reflector of the Householder
# QRs :117-121 / :175-176) computed by hand, each with a planted mistake the
# same check must reject.

EPS_DIV = np.float32(1e-7)


def _bad_div_unsigned(num, denom, eps=1e-7):
    """Planted mistake: a value clamp |d| -> eps that loses the sign."""
    d = np.float32(np.asarray(denom).reshape(()))
    safe = np.float32(eps) if abs(d) < eps else d
    return O._b(np.asarray(num, np.float32) / np.float32(safe))


def _bad_div_sign0(num, denom, eps=1e-7):
    """Planted mistake: sign(0) = 0, so a zero divisor stays zero."""
    d = np.float32(np.asarray(denom).reshape(()))
    safe = np.sign(d) * np.float32(eps) if abs(d) < eps else d
    with np.errstate(divide="ignore", invalid="ignore"):
        return O._b(np.asarray(num, np.float32) / np.float32(safe))


def test_safe_div_hand_cases():
    one = np.array([1.0], np.float32)
    cases = [
        (5e-8, 1e7),          # |d| < eps, positive: divide by +eps
        (-5e-8, -1e7),        # |d| < eps, negative: divide by -eps (sign kept)
        (0.0, 1e7),           # sign(0) -> +1: divide by +eps
        (-0.0, 1e7),          # -0.0 == 0 as well: +eps
        (1e-7, 1e7),          # |d| == eps is not clamped (and divides alike)
        (2.0, 0.5),           # ordinary divisor
        (-4.0, -0.25),
    ]
    for d, want in cases:
        got = float(O._safe_div(one, np.float32(d))[0])
        assert got == float(O.bf16_round(np.array([want], np.float32))[0]), (d, got)
    assert np.isnan(O._safe_div(one, np.float32(np.nan))[0])   # NaN divisor propagates
    # the checks reject an unsigned clamp and a sign(0) = 0 clamp
    assert float(_bad_div_unsigned(one, np.float32(-5e-8))[0]) > 0
    with np.errstate(divide="ignore", invalid="ignore"):
        assert not np.isfinite(_bad_div_sign0(one, np.float32(0.0))[0])


def _bad_chol_clamp0(A):
    """Planted mistake: the pivot clamped at 0 instead of 1e-7."""
    A = O._b(A)
    n = A.shape[0]
    L = np.zeros_like(A)
    for j in range(n):
        ss = np.float32((L[j, :j].astype(np.float32) ** 2).sum())
        L[j, j] = O._b(np.sqrt(np.float32(max(np.float32(A[j, j]) - ss, np.float32(0.0)))))
        if j + 1 < n:
            head = O._mm(L[j + 1:, :j], L[j:j + 1, :j].T)
            with np.errstate(divide="ignore", invalid="ignore"):
                L[j + 1:, j:j + 1] = O._b((O._b(A[j + 1:, j:j + 1] - head)) / L[j, j])
    return L


def test_cholesky_bf16_pivot_clamp_hand_cases():
    r = float(O.bf16_round(np.array([math.sqrt(1e-7)], np.float32))[0])   # bf16(sqrt(1e-7))
    # singular (rank 1): every pivot after the first is 0 -> sqrt(1e-7), and the
    # columns below them are exactly 0
    u = np.array([1.0, 2.0, -3.0, 1.0], np.float32)
    L = O.cholesky_bf16(np.outer(u, u))
    want = np.diag([1.0, r, r, r]).astype(np.float32)
    want[:, 0] = u
    assert np.array_equal(L, want)
    # indefinite: a negative pivot is clamped, later pivots are exact
    L = O.cholesky_bf16(np.array([[4.0, 2.0, 0.0], [2.0, -3.0, 0.0], [0.0, 0.0, 9.0]], np.float32))
    assert np.array_equal(L, np.array([[2.0, 0, 0], [1.0, r, 0], [0, 0, 3.0]], np.float32))
    # a NaN pivot propagates (torch's clamp_min keeps NaN) through everything below it
    A = np.eye(3, dtype=np.float32)
    A[0, 0] = np.nan
    L = O.cholesky_bf16(A)
    assert np.isnan(L[np.tril_indices(3)]).all()
    # the planted clamp-at-zero gives a zero pivot, which the hand case rejects
    with np.errstate(divide="ignore", invalid="ignore"):
        bad = _bad_chol_clamp0(np.outer(u, u))
    assert not np.array_equal(bad, want)


def test_householder_qr_bf16_zero_and_sign_cases():
    # a column that is zero from the diagonal down: zero-norm reflector, skipped
    A = np.array([[1.0, 0.0], [0.0, 0.0], [0.0, 0.0]], np.float32)
    R = O.householder_qr_bf16(A)
    assert np.array_equal(R, np.array([[-1.0, 0.0], [0.0, 0.0]], np.float32))
    # the reflector sign is -sign(x0) with torch's sign(0) = 0: a column whose
    # leading entry is exactly 0 gets alpha = 0, and v = x / ||x|| reflects x to
    # -x instead of onto e1, so R's diagonal entry stays 0
    A = np.array([[0.0, 1.0], [3.0, 1.0], [4.0, 1.0]], np.float32)
    R = O.householder_qr_bf16(A)
    assert R[0, 0] == 0.0 and R[0, 1] == 1.0
    assert abs(abs(float(R[1, 1])) - math.sqrt(0.68 ** 2 + 1.24 ** 2)) < 2e-2

    # planted mistake: sign(0) taken as +1 (the LAPACK convention) gives -5 there
    def qr_sign_plus(A):
        A = O._b(A).copy()
        m, n = A.shape
        for i in range(n):
            x = A[i:, i:i + 1]
            s = 1.0 if x[0, 0] >= 0 else -1.0
            alpha = -s * O._safe_norm(x)
            v = x.copy()
            v[0, 0] = O._b(v[0, 0] - alpha)
            vn = O._safe_norm(v)
            if vn == 0.0:
                continue
            v = O._safe_div(v, vn)
            blk = A[i:, i:]
            A[i:, i:] = O._b(blk - O._b(2.0 * O._mm(v, O._mm(v.T, blk))))
        return np.triu(A[:n, :n])
    assert qr_sign_plus(A)[0, 0] == -5.0

    # planted mistake: no zero-norm skip (v / 0) poisons the factor
    def qr_no_skip(A):
        A = O._b(A).copy()
        m, n = A.shape
        for i in range(n):
            x = A[i:, i:i + 1]
            alpha = -np.sign(x[0, 0]) * O._safe_norm(x)
            v = x.copy()
            v[0, 0] = O._b(v[0, 0] - alpha)
            with np.errstate(divide="ignore", invalid="ignore"):
                v = O._b(v / O._safe_norm(v))
                blk = A[i:, i:]
                A[i:, i:] = O._b(blk - O._b(2.0 * O._mm(v, O._mm(v.T, blk))))
        return np.triu(A[:n, :n])
    with np.errstate(invalid="ignore"):
        assert not np.isfinite(qr_no_skip(np.array([[1.0, 0.0], [0.0, 0.0], [0.0, 0.0]],
                                                  np.float32))).all()


def test_solve_triangular_bf16_tiny_and_zero_diagonals():
    """Back and forward substitution through the _safe_div clamp, by hand."""
    R = np.array([[2.0, 1.0], [0.0, 5e-8]], np.float32)
    X = O.solve_triangular_bf16(R, np.array([[1.0], [1.0]], np.float32), upper=True)
    x1 = float(O.bf16_round(np.array([1e7], np.float32))[0])
    assert X[1, 0] == x1
    assert X[0, 0] == float(O.bf16_round(np.array([(1.0 - x1) / 2.0], np.float32))[0])
    Rn = np.array([[2.0, 1.0], [0.0, -5e-8]], np.float32)   # sign kept
    assert O.solve_triangular_bf16(Rn, np.array([[1.0], [1.0]], np.float32))[1, 0] == -x1
    Rz = np.array([[0.0, 0.0], [3.0, 4.0]], np.float32)     # lower, zero pivot -> +1e-7
    X = O.solve_triangular_bf16(Rz, np.array([[1.0], [2.0]], np.float32), upper=False)
    assert X[0, 0] == x1
    # the unsigned-clamp mistake flips the sign of the negative case
    assert float(_bad_div_unsigned(np.array([1.0], np.float32), np.float32(-5e-8))[0]) == x1


# ---------------------------------------------------------------------------
# Classic K-FAC control (kfac_hooks.py / classic_kfac.py)
# ---------------------------------------------------------------------------
def test_gram_average_brute_force_and_chunking():
    rng = np.random.default_rng(41)
    chunks = [rng.standard_normal((r, 5)) for r in (3, 7, 1)]
    want = np.zeros((5, 5))
    for x in chunks:
        for row in x:
            for i in range(5):
                for j in range(5):
                    want[i, j] += row[i] * row[j]
    want /= 11
    got = O.gram_average(chunks)
    assert np.allclose(got, want, rtol=1e-13, atol=1e-14)
    # one chunk of all rows gives the same average
    assert np.allclose(O.gram_average([np.concatenate(chunks)]), want, rtol=1e-13)
    # planted mistake: averaging per chunk (1 / number of chunks) is rejected
    bad = sum(x.T @ x / x.shape[0] for x in chunks) / len(chunks)
    assert not np.allclose(bad, want, rtol=1e-3)


def test_classic_inverse_closed_forms():
    A = np.array([[4.0]])
    assert np.allclose(O.classic_inverse(A, 1.0), [[0.2]], rtol=1e-15)
    d = np.array([1.0, 3.0, 0.5])
    assert np.allclose(O.classic_inverse(np.diag(d), 0.5), np.diag(1 / (d + 0.5)), rtol=1e-15)
    rng = np.random.default_rng(2)
    X = rng.standard_normal((30, 6))
    A = X.T @ X / 30
    Xi = O.classic_inverse(A, 1e-2)
    assert np.allclose((A + 1e-2 * np.eye(6)) @ Xi, np.eye(6), atol=1e-12)
    # planted mistake: the undamped inverse fails the damped identity
    assert not np.allclose((A + 1e-2 * np.eye(6)) @ np.linalg.inv(A), np.eye(6), atol=1e-6)


def test_classic_nat_diagonal_closed_form():
    a = np.array([1.0, 2.0, 4.0])
    g = np.array([0.5, 3.0])
    lam = 0.1
    grad = np.arange(6.0).reshape(2, 3) + 1
    got = O.classic_nat(grad, O.classic_inverse(np.diag(a), lam), O.classic_inverse(np.diag(g), lam))
    want = grad / np.outer(g + lam, a + lam)
    assert np.allclose(got, want, rtol=1e-14)
    # the transposed product (A^{-1} on the left) would not even conform
    assert got.shape == (2, 3)


def test_classic_schedule_by_hand():
    assert [s for s in range(1, 8) if O.classic_updates_at(s, 1)] == list(range(1, 8))
    assert [s for s in range(1, 12) if O.classic_updates_at(s, 3)] == [1, 4, 7, 10]
    assert [s for s in range(1, 32) if O.classic_updates_at(s, 10)] == [1, 11, 21, 31]
    # IFKFAC's schedule differs: step % freq == 0 once step >= freq
    assert [s for s in range(1, 32) if O.should_update_factors(s, 10)] == [10, 20, 30]


# ---------------------------------------------------------------------------
# Laplace consumer (laplace.py)
# ---------------------------------------------------------------------------
def test_factor_evd_closed_forms():
    # diagonal R: eigenvalues r_ii^2 descending, eigenvectors the unit vectors
    V, d = O.factor_evd(np.diag([1.0, 3.0, 2.0]))
    assert np.allclose(d, [9.0, 4.0, 1.0], rtol=1e-14)
    assert np.allclose(np.abs(V), np.eye(3)[:, [1, 2, 0]], atol=1e-14)
    # 2 x 2: R = [[a, b], [0, c]], R^T R = [[a^2, ab], [ab, b^2 + c^2]]
    a, b, c = 2.0, 1.0, 1.0
    A = np.array([[a * a, a * b], [a * b, b * b + c * c]])
    tr, det = np.trace(A), np.linalg.det(A)
    lam = np.array([tr / 2 + math.sqrt(tr * tr / 4 - det), tr / 2 - math.sqrt(tr * tr / 4 - det)])
    V, d = O.factor_evd(np.array([[a, b], [0.0, c]]))
    assert np.allclose(d, lam, rtol=1e-14)
    # reconstruction, lower triangle ignored
    rng = np.random.default_rng(3)
    R = np.triu(rng.standard_normal((6, 6))) + 3 * np.eye(6)
    Rg = R + np.tril(rng.standard_normal((6, 6)), -1)
    V, d = O.factor_evd(Rg)
    assert np.allclose(V @ np.diag(d) @ V.T, R.T @ R, atol=1e-12)
    assert np.all(np.diff(d) <= 0)
    # planted mistake: the left singular vectors do not diagonalise R^T R
    U = np.linalg.svd(R)[0]
    assert not np.allclose(U @ np.diag(d) @ U.T, R.T @ R, atol=1e-6)


def test_laplace_scales_and_identity_basis_sample():
    s = O.laplace_scales(np.array([0.0, 1.0, 3.0]), 4, 9.0)
    assert np.allclose(s, [1 / math.sqrt(3.0), 1 / math.sqrt(5.0), 1 / 3.0], rtol=1e-15)
    Xi = np.arange(6.0).reshape(2, 3) - 2
    W0 = np.ones((2, 3))
    sG, sA = np.array([2.0, 0.5]), np.array([1.0, 3.0, 0.25])
    got = O.laplace_sample(W0, np.eye(3), sA, np.eye(2), sG, Xi)
    want = np.ones((2, 3)) + Xi * np.outer(sG, sA)
    assert np.allclose(got, want, rtol=1e-15)


def test_laplace_sample_kronecker_covariance():
    """Draws of vec(dW) (row-major) have covariance Sigma_G (x) Sigma_A with
    Sigma = U diag(s^2) U^T; swapping the two sides is rejected."""
    rng = np.random.default_rng(11)
    n_out, n_in, N = 2, 3, 60000
    U_G = np.linalg.qr(rng.standard_normal((n_out, n_out)))[0]
    U_A = np.linalg.qr(rng.standard_normal((n_in, n_in)))[0]
    s_G, s_A = np.array([1.5, 0.5]), np.array([1.0, 0.7, 0.2])
    W0 = np.zeros((n_out, n_in))
    Xi = rng.standard_normal((N, n_out, n_in))
    D = np.einsum("ij,njk,lk->nil", U_G * s_G, Xi, U_A * s_A).reshape(N, -1)
    cov = D.T @ D / N
    want = np.kron(U_G @ np.diag(s_G ** 2) @ U_G.T, U_A @ np.diag(s_A ** 2) @ U_A.T)
    assert np.abs(cov - want).max() < 0.03
    one = O.laplace_sample(W0, U_A, s_A, U_G, s_G, Xi[0]).reshape(-1)
    assert np.allclose(one, D[0], atol=1e-12)
    swapped = np.kron(U_A @ np.diag(s_A ** 2) @ U_A.T, U_G @ np.diag(s_G ** 2) @ U_G.T)
    assert np.abs(cov - swapped).max() > 0.1
