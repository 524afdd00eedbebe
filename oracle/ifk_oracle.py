"""CPU oracle for the IFKFAC curvature path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker or the timed CPU baseline; the
product (ifkfac_amd) never calls it.

Each function restates the reference algorithm (Gsend/ifkfac) in numpy and
cites the file:line it follows.  QR and triangular solves go through numpy /
scipy LAPACK (the same routine family the reference reaches through
torch.linalg on CPU).  How each function is pinned (tests/test_oracle.py):

  positive_diagonal          closed form; sign(0) = +1 special case
  gram_pivot_ratio           two columns at angle t: (1, sin^2 t) by hand;
                             orthogonal columns all 1; a repeated column 0
  streaming_tsqr_update      uniqueness: R^T R = sum X_i^T X_i with positive
                             diagonal == Cholesky factor of the Gram matrix;
                             exact-rational Gram-Schmidt on tiny integer inputs
  finalize_R / get_factors   R_d = chol(X^T X / rows + lambda I) (fp64)
  apply_vered(_bias)         (G + lambda I)^-1 grad (A + lambda I)^-1 closed form
                             and the recipe tests of tests/test_equivalence.py
  bf16_round                 hand-computed RNE ties, NaN/Inf, subnormals
  momentum_step              the recurrence unrolled by hand for 3 steps
  gram_average               brute-force sum of row outer products; chunking
                             invariance; a planted 1/chunks average fails
  classic_inverse            (A + lambda I) X = I; 1x1 and diagonal closed
                             forms; a planted undamped inverse fails
  classic_nat                diagonal closed form g_ij / ((a_j + l)(g_i + l))
  classic_updates_at         the schedule listed by hand for freq 1, 3, 10
  factor_evd                 diagonal and 2 x 2 closed forms; V diag(d) V^T =
                             R^T R; the lower triangle ignored; d descending;
                             a planted left-vector mistake fails
  laplace_scales             by hand
  laplace_sample             identity bases: elementwise by hand; the sample
                             covariance of many draws matches the Kronecker
                             covariance and rejects swapped sides
  bf16_linalg restatements   R vs chol(A^T A), L L^T vs A, R X vs B at tolerance;
                             the special cases by hand: _safe_div's signed
                             magnitude clamp (|d| < 1e-7 -> sign(d) 1e-7, sign(0)
                             = +1, NaN kept), cholesky_bf16's clamp_min(1e-7)
                             pivot (singular and indefinite inputs, NaN kept),
                             the zero-norm reflector skip and torch's sign(0) = 0
                             in the reflector sign, each with a planted mistake
                             the check rejects.  Bit-level parity of general
                             inputs: unpinned (the reference's bf16 matmul
                             rounding and accumulation order are not fixed by
                             any fixture the reference holds)
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import scipy.linalg as sla

# ----------------------------------------------------------------------------
# input generators (seeded; the kappa recipe of tests/test_bf16_stability.py:23-29)
# ----------------------------------------------------------------------------


def haar(m: int, k: int, rng: np.random.Generator) -> np.ndarray:
    """m x k matrix with Haar-distributed orthonormal columns (QR with sign fix)."""
    Q, R = np.linalg.qr(rng.standard_normal((m, k)))
    return Q * np.sign(np.diag(R))[None, :]


def kappa_matrix(p: int, n: int, kappa: float, rng: np.random.Generator) -> np.ndarray:
    """X = U diag(s) V^T, s log-spaced from 1 down to 1/kappa over min(p, n) values."""
    k = min(p, n)
    U = haar(p, k, rng)
    V = haar(n, k, rng)
    s = np.logspace(0.0, -math.log10(kappa), k)
    return (U * s[None, :]) @ V.T


# ----------------------------------------------------------------------------
# bf16 rounding (torch's .to(torch.bfloat16): round to nearest, ties to even)
# ----------------------------------------------------------------------------


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 -> fp32 with round-to-nearest-even, NaN kept NaN."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


# ----------------------------------------------------------------------------
# triangular.py restatements
# ----------------------------------------------------------------------------


def positive_diagonal(R: np.ndarray) -> np.ndarray:
    """Rows scaled by sign of their diagonal entry, sign 0 -> +1 (triangular.py:230-239)."""
    d = np.diag(R)[: R.shape[0]]
    s = np.sign(d)
    s[s == 0] = 1
    return R * s[:, None]


def _qr_r(A: np.ndarray) -> np.ndarray:
    """R of torch.linalg.qr(A, mode='reduced'): min(m, n) x n."""
    return np.linalg.qr(A, mode="r")


def streaming_tsqr_update(running_R: Optional[np.ndarray], new_chunk: np.ndarray) -> np.ndarray:
    """triangular.py:246-307: leaf QR of the chunk, then QR of [R_old; R_new]."""
    R_new = _qr_r(new_chunk)
    if running_R is None:
        return positive_diagonal(R_new)
    return positive_diagonal(_qr_r(np.vstack([running_R, R_new])))


def gram_pivot_ratio(P: np.ndarray) -> np.ndarray:
    """Pivot ratios of the Cholesky of A = P^T P: R_kk^2 / A_kk for each column,
    the squared sine of the angle between column k and the span of the columns
    before it.  No counterpart in the reference: it is the rule by which the
    Gram-route fold (ifk_tsqr_fold_gram) refuses a chunk and the panel fold
    (triangular.py:246-307) takes it instead.  Computed from the QR of P (fp64),
    so the checker itself does not lose the small ratios to the Gram matrix."""
    R = _qr_r(np.asarray(P, dtype=np.float64))
    d = np.sum(np.asarray(P, dtype=np.float64) ** 2, axis=0)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(d > 0, np.diag(R) ** 2 / np.where(d > 0, d, 1.0), 0.0)


def finalize_R(running_R: np.ndarray, damping: float) -> np.ndarray:
    """triangular.py:386-421: QR of [R; sqrt(damping) I], positive diagonal."""
    n = running_R.shape[0]
    return positive_diagonal(_qr_r(np.vstack([running_R, math.sqrt(damping) * np.eye(n)])))


def get_factor(R_raw: Optional[np.ndarray], rows: int, damping: float) -> Optional[np.ndarray]:
    """One side of get_factors (activation_hooks.py:262-332): None if no data or
    non-square (p < n), else finalize_R(R_raw / sqrt(rows), damping)."""
    if R_raw is None or R_raw.shape[0] != R_raw.shape[1]:
        return None
    return finalize_R(R_raw / math.sqrt(rows), damping)


def apply_vered(grad_W: np.ndarray, R_X: np.ndarray, R_G: np.ndarray) -> np.ndarray:
    """triangular.py:630-651: four triangular solves, in the dtype of the inputs."""
    T1 = sla.solve_triangular(R_G.T, grad_W, lower=True)
    T2 = sla.solve_triangular(R_G, T1, lower=False)
    T3_T = sla.solve_triangular(R_X.T, T2.T, lower=True)
    T4_T = sla.solve_triangular(R_X, T3_T, lower=False)
    return T4_T.T


def apply_vered_bias(grad_b: np.ndarray, R_G: np.ndarray) -> np.ndarray:
    """triangular.py:699-702: G^-1 g_b by two solves."""
    t = sla.solve_triangular(R_G.T, grad_b, lower=True)
    return sla.solve_triangular(R_G, t, lower=False)


def natgrad_closed_form(X: np.ndarray, dY: np.ndarray, grad_W: np.ndarray,
                        damping: float) -> np.ndarray:
    """(G + lambda I)^-1 grad (A + lambda I)^-1 with A = X^T X / p, G = dY^T dY / p
    (tests/test_equivalence.py:19-30), fp64."""
    p = X.shape[0]
    A = X.T @ X / p + damping * np.eye(X.shape[1])
    G = dY.T @ dY / p + damping * np.eye(dY.shape[1])
    return np.linalg.solve(G, grad_W) @ np.linalg.inv(A)


def chol_factor(Xs, rows: int, damping: float) -> np.ndarray:
    """Closed form of the damped factor: upper Cholesky of sum X^T X / rows + lambda I."""
    n = Xs[0].shape[1]
    A = sum(X.astype(np.float64).T @ X.astype(np.float64) for X in Xs) / rows
    A = A + damping * np.eye(n)
    return np.linalg.cholesky(A).T


# ----------------------------------------------------------------------------
# ifkfac.py restatements
# ----------------------------------------------------------------------------


def momentum_step(nat: np.ndarray, buf: Optional[np.ndarray], W: np.ndarray, lr: float,
                  momentum: float, weight_decay: float) -> Tuple[np.ndarray, Optional[np.ndarray]]:
    """ifkfac.py:402-413 in fp32 with the reference's operation order.
    Returns (W_new, buf_new); buf None means the buffer does not exist yet."""
    f = np.float32
    nat = nat.astype(f)
    W = W.astype(f).copy()
    if momentum > 0:
        if buf is None:
            buf = np.zeros_like(nat)
        buf = (buf * f(momentum)).astype(f) + nat
        d = buf
    else:
        d = nat
    if weight_decay > 0:
        W = (W * f(1.0 - lr * weight_decay)).astype(f)
    W = (W + f(-lr) * d).astype(f)
    return W, buf


def should_update_factors(step: int, freq: int) -> bool:
    """Schedule of IFKFAC.step (ifkfac.py:560-564)."""
    if freq == 1:
        return True
    return step >= freq and step % freq == 0


# ----------------------------------------------------------------------------
# kfac_hooks.py / classic_kfac.py restatements (the Classic K-FAC control)
# ----------------------------------------------------------------------------


def gram_average(chunks) -> np.ndarray:
    """A = sum_i x_i^T x_i / sum_i rows_i over the captured chunks
    (kfac_hooks.py:208-214 accumulate, :262-264 average), in fp64."""
    S = None
    rows = 0
    for x in chunks:
        x = np.asarray(x, dtype=np.float64)
        g = x.T @ x
        S = g if S is None else S + g
        rows += x.shape[0]
    return S / rows


def classic_inverse(A: np.ndarray, damping: float) -> np.ndarray:
    """(A + damping I)^{-1} by LU, torch.linalg.inv's method (classic_kfac.py:131-138)."""
    A = np.asarray(A, dtype=np.float64)
    return np.linalg.inv(A + damping * np.eye(A.shape[0]))


def classic_nat(grad_W: np.ndarray, A_inv: np.ndarray, G_inv: np.ndarray) -> np.ndarray:
    """G^{-1} grad A^{-1} (classic_kfac.py:218)."""
    return np.asarray(G_inv, np.float64) @ np.asarray(grad_W, np.float64) @ \
        np.asarray(A_inv, np.float64)


def classic_updates_at(step: int, freq: int) -> bool:
    """ClassicKFAC's schedule (classic_kfac.py:154,158): step % freq == 1, or every
    step when freq == 1 -- one step after IFKFAC's step % freq == 0."""
    return freq == 1 or step % freq == 1


# ----------------------------------------------------------------------------
# laplace.py restatements (the Laplace consumer of the factors)
# ----------------------------------------------------------------------------


def factor_evd(R: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """(V, d) with R^T R = V diag(d) V^T, d descending: the right singular vectors
    and squared singular values of the upper triangle of R -- svd(R), the
    IFKFAC route of laplace.py:26-30 (README.md:167 names it factors_to_evd)."""
    R = np.triu(np.asarray(R, dtype=np.float64))
    _, s, Vh = np.linalg.svd(R)
    return Vh.T, s * s


def laplace_scales(d: np.ndarray, dataset_size: int, prior_precision: float) -> np.ndarray:
    """1 / sqrt(sqrt(N) d + sqrt(lambda)) (laplace.py:92-101)."""
    return 1.0 / np.sqrt(math.sqrt(dataset_size) * np.asarray(d, np.float64) +
                         math.sqrt(prior_precision))


def laplace_sample(W_map: np.ndarray, U_A: np.ndarray, s_A: np.ndarray, U_G: np.ndarray,
                   s_G: np.ndarray, Xi: np.ndarray) -> np.ndarray:
    """W_map + U_G diag(s_G) Xi diag(s_A) U_A^T (laplace.py:138-154)."""
    xs = np.asarray(Xi, np.float64) * np.asarray(s_G, np.float64)[:, None] * \
        np.asarray(s_A, np.float64)[None, :]
    return np.asarray(W_map, np.float64) + np.asarray(U_G, np.float64) @ xs @ \
        np.asarray(U_A, np.float64).T


# ----------------------------------------------------------------------------
# bf16_linalg.py restatements (bf16 storage emulated by rounding every
# produced tensor; matmuls accumulate in fp32 then round)
# ----------------------------------------------------------------------------


def _b(x):
    a = np.asarray(x, dtype=np.float32)
    return bf16_round(a).reshape(a.shape)


def _mm(a, b):
    return _b(np.asarray(a, np.float32) @ np.asarray(b, np.float32))


def _safe_norm(x):
    return _b(np.linalg.norm(np.asarray(x, np.float32).astype(np.float32)))


def _safe_div(num, denom, eps=1e-7):
    d = np.float32(np.asarray(denom).reshape(()))
    s = np.sign(d) if d != 0 else np.float32(1.0)
    safe = s * np.float32(eps) if abs(d) < eps else d
    return _b(np.asarray(num, np.float32) / np.float32(safe))


def householder_qr_bf16(A: np.ndarray) -> np.ndarray:
    """bf16_linalg.py:158-183 (unblocked), small sizes only."""
    A = _b(A).copy()
    m, n = A.shape
    for i in range(n):
        x = A[i:, i:i + 1]
        alpha = -np.sign(x[0, 0]) * _safe_norm(x)
        v = x.copy()
        v[0, 0] = _b(v[0, 0] - alpha)
        vn = _safe_norm(v)
        if vn == 0.0:
            continue
        v = _safe_div(v, vn)
        blk = A[i:, i:]
        coeffs = _mm(v.T, blk)
        A[i:, i:] = _b(blk - _b(2.0 * _mm(v, coeffs)))
    return np.triu(A[:n, :n])


def solve_triangular_bf16(R: np.ndarray, B: np.ndarray, upper: bool = True) -> np.ndarray:
    """bf16_linalg.py:223-241: row-by-row substitution with _safe_div."""
    R = _b(R)
    B = _b(B)
    n = R.shape[0]
    X = np.zeros_like(B)
    rng = range(n - 1, -1, -1) if upper else range(n)
    for i in rng:
        if upper and i + 1 < n:
            rhs = _b(B[i:i + 1] - _mm(R[i:i + 1, i + 1:], X[i + 1:]))
        elif (not upper) and i > 0:
            rhs = _b(B[i:i + 1] - _mm(R[i:i + 1, :i], X[:i]))
        else:
            rhs = B[i:i + 1]
        X[i:i + 1] = _safe_div(rhs, R[i, i])
    return X


def cholesky_bf16(A: np.ndarray) -> np.ndarray:
    """bf16_linalg.py:247-267: pivots max(., 1e-7) in fp32."""
    A = _b(A)
    n = A.shape[0]
    L = np.zeros_like(A)
    for j in range(n):
        ss = np.float32((L[j, :j].astype(np.float32) ** 2).sum())
        piv = np.float32(np.float32(A[j, j]) - ss)
        # torch's clamp_min(1e-7) (bf16_linalg.py:258): NaN stays NaN
        d = piv if (np.isnan(piv) or piv >= np.float32(1e-7)) else np.float32(1e-7)
        L[j, j] = _b(np.sqrt(d))
        if j + 1 < n:
            below = A[j + 1:, j:j + 1]
            head = _mm(L[j + 1:, :j], L[j:j + 1, :j].T)
            L[j + 1:, j:j + 1] = _safe_div(_b(below - head), L[j, j])
    return L


def inv_spd_bf16(A: np.ndarray) -> np.ndarray:
    """bf16_linalg.py:272-280."""
    L = cholesky_bf16(A)
    n = A.shape[0]
    Y = solve_triangular_bf16(L, np.eye(n, dtype=np.float32), upper=False)
    return solve_triangular_bf16(np.ascontiguousarray(L.T), Y, upper=True)
