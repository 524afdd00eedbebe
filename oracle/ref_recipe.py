"""The reference's CPU call sequence, restated on torch CPU -- TEST / BASELINE ONLY.

Issues the same torch library calls, in the same order, as the reference's
curvature path does on host tensors, so that the CPU baseline of bench.py
times the algorithm the reference runs (LAPACK geqrf+orgqr through
torch.linalg.qr, LAPACK trsm through torch.linalg.solve_triangular):

  fold          triangular.py:284 (leaf qr), :299-301 (cat + merge qr), :230-239
  scale         activation_hooks.py:328-329
  finalize      triangular.py:411-416
  bf16 cast     ifkfac.py:292-294
  4 solves      triangular.py:621-628 (bf16 factors) / :632-651 (fp32 factors)
  momentum      ifkfac.py:404-413

Only tests/ and bench.py's cpu_baseline leg use this module.
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def positive_diagonal(R: torch.Tensor) -> torch.Tensor:
    signs = R.diag().sign()
    signs[signs == 0] = 1
    return R * signs.unsqueeze(1)


def fold(running_R: Optional[torch.Tensor], chunk: torch.Tensor) -> torch.Tensor:
    _, R_new = torch.linalg.qr(chunk, mode="reduced")
    if running_R is None:
        return positive_diagonal(R_new)
    _, R_m = torch.linalg.qr(torch.cat([running_R, R_new], dim=0), mode="reduced")
    return positive_diagonal(R_m)


def finalize(running_R: torch.Tensor, damping: float) -> torch.Tensor:
    n = running_R.shape[0]
    damp = (damping ** 0.5) * torch.eye(n, dtype=running_R.dtype)
    _, R = torch.linalg.qr(torch.cat([running_R, damp], dim=0), mode="reduced")
    return positive_diagonal(R)


def apply_vered(grad_W: torch.Tensor, R_X: torch.Tensor, R_G: torch.Tensor) -> torch.Tensor:
    if R_X.dtype == torch.bfloat16 or R_G.dtype == torch.bfloat16:
        RX, RG, g = R_X.float(), R_G.float(), grad_W.float()
        T1 = torch.linalg.solve_triangular(RG.t(), g, upper=False)
        T2 = torch.linalg.solve_triangular(RG, T1, upper=True)
        T3_T = torch.linalg.solve_triangular(RX.t(), T2.t(), upper=False)
        T4_T = torch.linalg.solve_triangular(RX, T3_T, upper=True)
        return T4_T.t().contiguous().to(grad_W.dtype)
    T1 = torch.linalg.solve_triangular(R_G.T, grad_W, upper=False)
    T2 = torch.linalg.solve_triangular(R_G, T1, upper=True)
    T3_T = torch.linalg.solve_triangular(R_X.T, T2.T, upper=False)
    T4_T = torch.linalg.solve_triangular(R_X, T3_T, upper=True)
    return T4_T.T


def factor_update_precond_step(X_chunks, D_chunks, grad_W: torch.Tensor, W: torch.Tensor,
                               buf: Optional[torch.Tensor], lr: float, momentum: float,
                               damping: float, use_true_bf16: bool):
    """One factor update plus one preconditioned step for a single layer.

    Returns (W, buf, R_X, R_G) after the step.  Mirrors the hooks' folds, then
    _update_factors, then the fast-path per-layer update of IFKFAC.step.
    """
    R_X = None
    R_G = None
    rows_X = rows_G = 0
    for X in X_chunks:
        R_X = fold(R_X, X)
        rows_X += X.shape[0]
    for D in D_chunks:
        R_G = fold(R_G, D)
        rows_G += D.shape[0]
    R_X = finalize(R_X / math.sqrt(rows_X), damping)
    R_G = finalize(R_G / math.sqrt(rows_G), damping)
    if use_true_bf16:
        R_X = R_X.to(torch.bfloat16)
        R_G = R_G.to(torch.bfloat16)
    nat = apply_vered(grad_W, R_X, R_G)
    if momentum > 0:
        if buf is None:
            buf = torch.zeros_like(nat)
        buf.mul_(momentum).add_(nat)
        nat = buf
    W.add_(nat, alpha=-lr)
    return W, buf, R_X, R_G
