"""Numerical seams of the IFKFAC curvature path, dispatched to the HIP library.

Same functions, argument meaning and fallback behaviour as the reference's
``ifkfac/triangular.py``; the arithmetic runs in the kernels behind
include/ifkfac_hip.h:

* ``streaming_tsqr_update`` (triangular.py:246-307) -> ``ifk_tsqr_fold``
* ``finalize_R``            (triangular.py:386-421) -> ``ifk_finalize``
* ``apply_vered``           (triangular.py:551-656) -> ``ifk_precondition``
* ``apply_vered_batched``   (triangular.py:506-544) -> bf16 factors: the
  inverses, then ``ifk_precondition_apply_bf16_batched`` (every product once
  over the bucket); fp32 factors: ``ifk_precondition`` per entry
* ``apply_vered_bias``      (triangular.py:659-705) -> two ``ifk_trsm``
* ``batched_streaming_tsqr_update`` (triangular.py:331-379) -> bf16
  arithmetic: ``ifk_tsqr_fold_gram_batched`` (one chain for the bucket, a
  refused entry by ``ifk_tsqr_fold``); fp32: ``ifk_tsqr_fold`` per entry
* ``tsqr``  (triangular.py:150-227) -> ``ifk_tsqr_fold`` over tiles of
  ``tile_size`` rows (the R factor of a full-rank matrix is unique, so the
  streamed tiles give the tree's R)
* ``sgso``  (triangular.py:89-143, the reference's test cross-check) -> the
  fold's R and Q = M R^{-1} by ``ifk_trsm``

Arithmetic modes: fp32 factors are handled with fp32 MFMA.  bf16 factors (the
``use_true_bf16`` storage) are handled with bf16 MFMA and fp32 accumulation
unless ``IFKFAC_BF16_SOLVE_MATH=f32`` is set in the environment, which keeps
fp32 arithmetic on the bf16-valued factors as the reference does.
"""
from __future__ import annotations

import logging
import os
from typing import Optional

import torch

from ._backend import MATH_BF16, MATH_F32, get_backend

logger = logging.getLogger(__name__)


def _bf16_solve_math() -> int:
    return MATH_F32 if os.environ.get("IFKFAC_BF16_SOLVE_MATH", "").lower() == "f32" else MATH_BF16


def solve_math_for(dtype: torch.dtype) -> int:
    """MFMA arithmetic used for factors of this storage dtype."""
    return _bf16_solve_math() if dtype == torch.bfloat16 else MATH_F32


def _positive_diagonal_R(R: torch.Tensor) -> torch.Tensor:
    """Scale each row of R by the sign of its diagonal entry (sign 0 -> +1)."""
    signs = R.diagonal().sign()
    signs = torch.where(signs == 0, torch.ones_like(signs), signs)
    return R * signs.unsqueeze(1)


def streaming_tsqr_update(running_R: Optional[torch.Tensor], new_chunk: torch.Tensor, *,
                          math: int = MATH_F32) -> torch.Tensor:
    """Fold one chunk of rows into the running R factor.

    ``running_R`` is None (no data yet) or the ``(r, n)`` upper-trapezoidal
    factor from earlier calls; ``new_chunk`` is ``(p_i, n)``.  Returns the
    ``(min(r + p_i, n), n)`` factor of ``[running_R; new_chunk]`` with a
    positive diagonal (a fresh tensor, fp32).
    """
    p, n = new_chunk.shape
    buf = torch.zeros((n, n), dtype=torch.float32, device=new_chunk.device)
    r_in = 0
    if running_R is not None:
        r_in = running_R.shape[0]
        if running_R.shape[1] != n:
            raise ValueError(f"running_R has {running_R.shape[1]} columns, chunk has {n}")
        buf[:r_in].copy_(running_R)
    r_new = get_backend().fold_(buf, r_in, new_chunk, math)
    return buf[:r_new]


def batched_streaming_tsqr_update(running_R: torch.Tensor, new_chunks: torch.Tensor, *,
                                  math: int = MATH_F32) -> torch.Tensor:
    """Fold ``new_chunks[i]`` into ``running_R[i]`` for every layer of a bucket.

    ``running_R`` is ``(B, n, n)`` (zeros for layers without data); chunks are
    ``(B, p, n)``, zero-padded along p.  Zero rows contribute nothing.  In bf16
    arithmetic the bucket goes through one batched Gram-route fold; an entry
    it refuses (status 2: its pivot test found the rows too ill-conditioned,
    its factor untouched) is folded by the panel path in fp32 arithmetic.
    """
    B, p, n = new_chunks.shape
    assert running_R.shape == (B, n, n), \
        f"running_R shape {tuple(running_R.shape)} != ({B}, {n}, {n})"
    be = get_backend()
    out = running_R.detach().to(torch.float32, copy=True).contiguous()
    if math == MATH_BF16 and B > 1 and hasattr(be, "fold_gram_batched_"):
        from .activation_hooks import GRAM_FOLD_TOL
        views = [out[i] for i in range(B)]
        chunks = [new_chunks[i] for i in range(B)]
        st = be.fold_gram_batched_(views, n, chunks, GRAM_FOLD_TOL).cpu()
        for i in range(B):
            if int(st[i]) != 1:
                be.fold_(views[i], n, chunks[i], MATH_F32)
        return out
    for i in range(B):
        be.fold_(out[i], n, new_chunks[i], math)
    return out


def tsqr(M: torch.Tensor, tile_size: int = 512) -> torch.Tensor:
    """R factor (positive diagonal) of a tall ``(p, n)`` matrix, ``p >= n``,
    folded ``tile_size`` rows at a time (the reference's leaf size)."""
    p, n = M.shape
    if p < n:
        raise ValueError(
            f"tsqr requires p >= n (got p={p}, n={n}).  "
            "IFKFAC needs batch_size × seq_len >= layer_input_dim.")
    if tile_size < 1:
        raise ValueError(f"tsqr: tile_size must be positive (got {tile_size})")
    be = get_backend()
    buf = torch.zeros((n, n), dtype=torch.float32, device=M.device)
    r = 0
    for r0 in range(0, p, tile_size):
        r = be.fold_(buf, r, M[r0:r0 + tile_size], MATH_F32)
    return buf


def sgso(M: torch.Tensor):
    """(Q, R) of a tall ``(p, n)`` matrix, ``p >= n``: R upper triangular with
    a positive diagonal and Q = M R^{-1} with orthonormal columns (the
    reference's Gram-Schmidt cross-check; for a full-rank M the pair is
    unique, so it is computed here from the fold's R and one triangular
    solve).  A column that is numerically zero after the earlier ones (a
    diagonal of R below 1e-12) is reported with the reference's warning and
    its diagonal taken as 1, as the reference's loop does."""
    import warnings
    p, n = M.shape
    if p < n:
        raise ValueError(
            f"sgso requires p >= n (got p={p}, n={n}).  "
            "IFKFAC needs batch_size × seq_len >= layer_input_dim.")
    R = tsqr(M, tile_size=max(p, 1))
    d = R.diagonal()
    small = (d.abs() < 1e-12).nonzero().flatten().tolist()
    for j in small:
        warnings.warn(
            f"sgso: column {j} is near-zero after deflation "
            f"(norm={float(d[j]):.2e}).  Matrix may be rank-deficient.",
            RuntimeWarning, stacklevel=2)
        R[j, j] = 1.0
    QT = get_backend().trsm(R.t().contiguous(), M.t().contiguous().float(), False,
                            torch.float32, MATH_F32)
    return QT.t().to(M.dtype), R.to(M.dtype)


def finalize_R(running_R: torch.Tensor, damping: float, *, math: int = MATH_F32) -> torch.Tensor:
    """Return R_d with R_d^T R_d = running_R^T running_R + damping * I."""
    R, _ = get_backend().finalize(running_R, 1.0, damping, torch.float32, math)
    return R


def apply_vered(grad_W: torch.Tensor, R_X: torch.Tensor, R_G: torch.Tensor) -> torch.Tensor:
    """Natural gradient ``(R_G^T R_G)^{-1} grad_W (R_X^T R_X)^{-1}``."""
    if R_X.dtype == torch.bfloat16 or R_G.dtype == torch.bfloat16:
        if R_X.shape[0] != R_X.shape[1]:
            print(f"[apply_vered bf16] SKIP — R_X non-square: "
                  f"shape={tuple(R_X.shape)}.  Returning raw gradient.", flush=True)
            return grad_W
        if R_G.shape[0] != R_G.shape[1]:
            print(f"[apply_vered bf16] SKIP — R_G non-square: "
                  f"shape={tuple(R_G.shape)}.  Returning raw gradient.", flush=True)
            return grad_W
        nat = get_backend().precondition(grad_W, R_X, R_G, _bf16_solve_math())
        return nat.to(grad_W.dtype)
    nat = get_backend().precondition(grad_W, R_X, R_G, MATH_F32)
    return nat if nat.dtype == grad_W.dtype else nat.to(grad_W.dtype)


def apply_vered_batched(grad_W: torch.Tensor, R_X: torch.Tensor, R_G: torch.Tensor) -> torch.Tensor:
    """``apply_vered`` over a bucket: grad_W (B, n_out, n_in), factors (B, n, n).

    bf16 factors in bf16 arithmetic: each entry's two triangular inverses,
    then every product of the four solves once over the whole bucket
    (``ifk_precondition_apply_bf16_batched``, each entry bit for bit its own
    ``precondition_apply_bf16``); otherwise ``apply_vered`` per entry."""
    B = grad_W.shape[0]
    assert R_X.shape[0] == B and R_G.shape[0] == B, \
        f"batch dims mismatch: grad_W={grad_W.shape[0]}, R_X={R_X.shape[0]}, R_G={R_G.shape[0]}"
    be = get_backend()
    square = R_X.shape[1] == R_X.shape[2] and R_G.shape[1] == R_G.shape[2]
    if (B > 1 and square and R_X.dtype == torch.bfloat16 and R_G.dtype == torch.bfloat16 and
            _bf16_solve_math() == MATH_BF16 and hasattr(be, "precondition_apply_bf16_batched")):
        # each side's copies stacked: the batched apply reads the bucket's
        # entries at one stride
        zx = [be.tri_inverse_bf16(R_X[i])[1:] for i in range(B)]
        zg = [be.tri_inverse_bf16(R_G[i])[1:] for i in range(B)]
        ZXb, ZXt = torch.stack([z[0] for z in zx]), torch.stack([z[1] for z in zx])
        ZGb, ZGt = torch.stack([z[0] for z in zg]), torch.stack([z[1] for z in zg])
        nat = be.precondition_apply_bf16_batched([grad_W[i] for i in range(B)],
                                                 [(ZXb[i], ZXt[i]) for i in range(B)],
                                                 [(ZGb[i], ZGt[i]) for i in range(B)])
        return nat.to(grad_W.dtype)
    return torch.stack([apply_vered(grad_W[i], R_X[i], R_G[i]) for i in range(B)], dim=0)


def apply_vered_bias(grad_b: torch.Tensor, R_G: torch.Tensor) -> torch.Tensor:
    """``(R_G^T R_G)^{-1} grad_b`` for a bias gradient of length n_out."""
    if R_G.dtype == torch.bfloat16 and R_G.shape[0] != R_G.shape[1]:
        print(f"[apply_vered_bias bf16] SKIP — R_G non-square: "
              f"shape={tuple(R_G.shape)}.  Returning raw bias gradient.", flush=True)
        return grad_b
    # two triangular solves, R_G^T y = g then R_G x = y (triangular.py:695-701),
    # in fp32 arithmetic on the (upcast) factor
    be = get_backend()
    g = grad_b.reshape(-1, 1).float()
    y = be.trsm(R_G.t(), g, False, torch.float32, MATH_F32)
    x = be.trsm(R_G, y, True, torch.float32, MATH_F32)
    return x.reshape(grad_b.shape).to(grad_b.dtype)
