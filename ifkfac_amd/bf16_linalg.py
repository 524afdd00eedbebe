"""bf16 linear-algebra primitives on the HIP kernels.

Counterparts of the reference's ``ifkfac/bf16_linalg.py`` with the same
names, argument meaning and input guards.  Storage is bf16; the contractions
run on bf16 MFMA with fp32 accumulation, reductions, divisors and pivots are
fp32, and results are rounded to bf16 once (RNE).  The reference rounds every
intermediate to bf16, so these results are at least as accurate; parity is at
the level of the reference's own checks (R against the Cholesky factor of
A^T A after sign normalisation, L L^T against A, R X against B).

Deliberate differences: the R factors are returned with a positive
diagonal (the reference leaves the Householder sign -sign(x0) on each
diagonal entry); ``block_size`` is accepted but the panel width is the
kernel's own (64 columns); and a column whose leading entry is exactly 0 is
reduced as LAPACK's dlarfg does (sign(0) = +1).  The reference takes torch's
sign(0) = 0 there (bf16_linalg.py:114, :173), so its reflector maps that
column to its negative instead of onto e1 and leaves the column unreduced.
The clamps of ``_safe_div`` and of the Cholesky pivot are the reference's,
NaN pivots included.
"""
from __future__ import annotations

import torch

from ._backend import MATH_BF16, get_backend


def _safe_norm(x: torch.Tensor) -> torch.Tensor:
    """Frobenius norm in fp32, returned in x's dtype (bf16_linalg.py:38-41)."""
    return x.float().norm().to(x.dtype)


def _safe_div(num: torch.Tensor, denom: torch.Tensor, eps: float = 1e-7) -> torch.Tensor:
    """num / denom in fp32 with |denom| < eps replaced by sign(denom) * eps,
    sign(0) = +1; result in num's dtype (bf16_linalg.py:44-59)."""
    d = denom.float()
    sgn = torch.sign(d)
    sgn = torch.where(sgn == 0, torch.ones_like(sgn), sgn)
    safe = torch.where(d.abs() < eps, sgn * eps, d)
    return (num.float() / safe).to(num.dtype)


def block_householder_qr_bf16(A: torch.Tensor, block_size: int = 32) -> torch.Tensor:
    """R factor (n x n, bf16, upper triangular) of a tall bf16 matrix A (m >= n)."""
    assert A.dtype == torch.bfloat16, f"expected bf16 input, got {A.dtype}"
    m, n = A.shape
    assert m >= n, f"need m >= n, got ({m}, {n})"
    return get_backend().geqrf_r(A, torch.bfloat16, MATH_BF16)


def householder_qr_bf16(A: torch.Tensor) -> torch.Tensor:
    """Unblocked-API variant of :func:`block_householder_qr_bf16` (same result)."""
    assert A.dtype == torch.bfloat16, f"expected bf16 input, got {A.dtype}"
    m, n = A.shape
    assert m >= n, f"need m >= n, got ({m}, {n})"
    return get_backend().geqrf_r(A, torch.bfloat16, MATH_BF16)


def solve_triangular_bf16(R: torch.Tensor, B: torch.Tensor, upper: bool = True) -> torch.Tensor:
    """Solve R X = B (R n x n triangular, B n x k, both bf16); returns bf16 X."""
    if R.dtype != torch.bfloat16 or B.dtype != torch.bfloat16:
        print(f"[bf16_linalg.solve_triangular_bf16] DTYPE MISMATCH: "
              f"R.dtype={R.dtype}, B.dtype={B.dtype}, "
              f"R.shape={tuple(R.shape)}, B.shape={tuple(B.shape)}", flush=True)
        raise TypeError(
            f"solve_triangular_bf16: both R and B must be bf16; "
            f"got R.dtype={R.dtype}, B.dtype={B.dtype}")
    if R.shape[1] != R.shape[0]:
        print(f"[bf16_linalg.solve_triangular_bf16] NON-SQUARE R: "
              f"R.shape={tuple(R.shape)}", flush=True)
        raise ValueError(f"R must be square, got {R.shape}")
    if B.shape[0] != R.shape[0]:
        print(f"[bf16_linalg.solve_triangular_bf16] SHAPE MISMATCH: "
              f"R.shape={tuple(R.shape)}, B.shape={tuple(B.shape)}", flush=True)
        raise ValueError(f"B rows must match R, got R={R.shape}, B={B.shape}")
    return get_backend().trsm(R, B, upper, torch.bfloat16, MATH_BF16)


def cholesky_bf16(A: torch.Tensor) -> torch.Tensor:
    """Lower L with L L^T = A for SPD bf16 A; pivots clamped at 1e-7."""
    assert A.dtype == torch.bfloat16
    return get_backend().potrf(A, torch.bfloat16, MATH_BF16)


def inv_spd_bf16(A: torch.Tensor) -> torch.Tensor:
    """A^{-1} for SPD bf16 A via its Cholesky factor; bf16 result."""
    return get_backend().inv_spd(A, torch.bfloat16, MATH_BF16)


def _self_test() -> None:
    """Print the relative errors of the primitives against fp32 references."""
    torch.manual_seed(0)
    device = torch.device("cuda")
    print(f"device: {device}\n")
    for n in (8, 32, 64, 256, 1000):
        A32 = torch.randn(2 * n, n, device=device)
        R = block_householder_qr_bf16(A32.bfloat16()).float()
        Rt = torch.linalg.cholesky((A32.double().t() @ A32.double())).t().float()
        print(f"  qr   n={n:>4d}  rel |R - chol(A^T A)| = "
              f"{((R - Rt).norm() / Rt.norm()).item():.3e}")
    for n in (8, 32, 64):
        R32 = torch.triu(torch.randn(n, n, device=device))
        R32 = R32 + torch.sign(torch.diagonal(R32)).diag()
        B32 = torch.randn(n, 4, device=device)
        X = solve_triangular_bf16(R32.bfloat16(), B32.bfloat16(), upper=True).float()
        Xt = torch.linalg.solve_triangular(R32, B32, upper=True)
        print(f"  trsm n={n:>3d}  rel = {((X - Xt).norm() / Xt.norm()).item():.3e}")
        Z = torch.randn(2 * n, n, device=device)
        S = Z.t() @ Z + torch.eye(n, device=device)
        L = cholesky_bf16(S.bfloat16()).float()
        Lt = torch.linalg.cholesky(S)
        print(f"  chol n={n:>3d}  rel = {((L - Lt).norm() / Lt.norm()).item():.3e}")
        Si = inv_spd_bf16(S.bfloat16()).float()
        St = torch.linalg.inv(S)
        print(f"  inv  n={n:>3d}  rel = {((Si - St).norm() / St.norm()).item():.3e}")


if __name__ == "__main__":
    _self_test()
