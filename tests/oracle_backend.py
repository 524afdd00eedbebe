"""Test double of ifkfac_amd's backend built on the CPU oracle.

Lets the CPU test suite drive the real host logic of ifkfac_amd (hooks,
schedule, skip/clear rules, classification, updates) without a GPU.  It is
installed only by tests (``_backend.set_backend``); the product never
constructs it.  Each method mirrors the HIP backend's contract on CPU tensors
and counts its calls so tests can assert how often each seam was used.
"""
from __future__ import annotations

import collections

import numpy as np
import scipy.linalg as sla
import torch

from oracle import ifk_oracle as O


def _np(t):
    return t.detach().to(torch.float64).cpu().numpy()


class OracleBackend:
    name = "oracle"

    def __init__(self):
        self.calls = collections.Counter()

    def fold_(self, R, r_in, X, math):
        self.calls["fold"] += 1
        n = R.shape[1]
        old = None if r_in == 0 else _np(R[:r_in])
        new = O.streaming_tsqr_update(old, _np(X))
        r_new = new.shape[0]
        R.zero_()
        R[:r_new] = torch.from_numpy(new).to(R.dtype)
        return r_new

    # tests set this to make the Gram-route fold refuse (status 2) once per call
    gram_fold_status2 = 0

    def fold_gram_(self, R, r_in, X, pivot_tol):
        """The Gram-route fold: status 2 (R untouched) when the Cholesky of the
        Gram matrix of [R[:r_in]; X] meets a pivot below pivot_tol of its column's
        diagonal (O.gram_pivot_ratio), else the fold's factor and status 1."""
        self.calls["fold_gram"] += 1
        n = R.shape[1]
        assert r_in + X.shape[0] >= n, "Gram-route fold of a partial-rank factor"
        old = None if r_in == 0 else _np(R[:r_in])
        P = _np(X) if old is None else np.vstack([old, _np(X)])
        if self.gram_fold_status2 > 0:
            self.gram_fold_status2 -= 1
            return torch.tensor([2], dtype=torch.int32)
        if not np.all(np.isfinite(P)):
            return torch.tensor([2], dtype=torch.int32)
        if O.gram_pivot_ratio(P).min() < pivot_tol:
            return torch.tensor([2], dtype=torch.int32)
        new = O.streaming_tsqr_update(old, _np(X))
        R.zero_()
        R[:n] = torch.from_numpy(new).to(R.dtype)
        return torch.tensor([1], dtype=torch.int32)

    def finalize(self, R, scale, damping, out_dtype, math):
        self.calls["finalize"] += 1
        Rd = O.finalize_R(_np(R) * scale, damping)
        out = torch.from_numpy(Rd).float().to(out_dtype)
        flag = torch.tensor([1 if np.all(np.isfinite(Rd)) else 0], dtype=torch.int32)
        return out, flag

    # tests set this to make the CholeskyQR2 variant report an ill-conditioned
    # block (status 2), as ifk_fold_finalize_cqr does, once per call
    cqr_status2 = 0

    def fold_finalize(self, R, r_in, X, scale, damping, out_dtype, math, cqr=False, gram=False,
                      with_kappa=False):
        """The fused fold + finalize; with cqr or gram the fast variants' status 2 can
        be injected (cqr_status2), and with_kappa returns the Gram path's kappa bound
        sqrt(1 + ||scale^2 P^T P||_F / damping) as a third value."""
        self.calls["fold_finalize"] += 1
        if cqr or gram:
            self.calls["fold_finalize_cqr" if cqr else "fold_finalize_gram"] += 1
            if self.cqr_status2 > 0:
                self.cqr_status2 -= 1
                n = X.shape[1]
                out = (torch.full((n, n), float("nan")).to(out_dtype),
                       torch.tensor([2], dtype=torch.int32))
                return out + (torch.tensor([float("inf")]),) if (gram and with_kappa) else out
        old = None if r_in == 0 else _np(R[:r_in])
        new = O.streaming_tsqr_update(old, _np(X))
        assert new.shape[0] == new.shape[1], "fused finalize of a partial-rank factor"
        Rd = O.finalize_R(new * scale, damping)
        out = torch.from_numpy(Rd).float().to(out_dtype)
        flag = torch.tensor([1 if np.all(np.isfinite(Rd)) else 0], dtype=torch.int32)
        if gram and with_kappa:
            E = scale * scale * (new.T @ new)
            kb = float(np.sqrt(1.0 + np.linalg.norm(E) / damping)) if damping > 0 else float("inf")
            return out, flag, torch.tensor([kb], dtype=torch.float32)
        return out, flag

    def fold_finalize_gram_batched(self, Rs, r_in, Xs, scale, damping, out_dtype,
                                   with_inverse=False):
        """The batched Gram factor update, entry by entry (the batched launch gives
        every entry the single call's bits).  With ``with_inverse`` also the
        inverse of each damped factor before its output rounding (fp64 here) and
        its bf16 copies, as ifk_fold_finalize_gram_inverse."""
        self.calls["fold_finalize_gram_batched"] += 1
        if with_inverse:
            self.calls["fold_finalize_gram_inverse"] += 1
        outs, sts, kbs, invs = [], [], [], []
        for e, X in enumerate(Xs):
            R = Rs[e] if Rs is not None else None
            o, s, k = self.fold_finalize(R, r_in, X, scale, damping, out_dtype, 1, gram=True,
                                         with_kappa=True)
            outs.append(o)
            sts.append(s)
            kbs.append(k)
            if with_inverse:
                old = None if r_in == 0 else _np(R[:r_in])
                Rd = O.finalize_R(O.streaming_tsqr_update(old, _np(X)) * scale, damping)
                Z = torch.from_numpy(np.linalg.inv(Rd)).float()
                if int(s.item()) == 2:
                    Z = torch.full_like(Z, float("nan"))
                invs.append(Z)
        if not with_inverse:
            return torch.stack(outs), torch.cat(sts), torch.cat(kbs)
        Z = torch.stack(invs)
        return (torch.stack(outs), torch.cat(sts), torch.cat(kbs),
                (Z, Z.bfloat16(), Z.transpose(1, 2).contiguous().bfloat16()))

    def tri_inverse(self, R, math):
        self.calls["tri_inverse"] += 1
        return torch.from_numpy(np.linalg.inv(_np(R))).float()

    def tri_inverse_bf16(self, R):
        """Z (fp32) and its RNE bf16 copies (Z, Z^T), as ifk_tri_inverse_bf16."""
        self.calls["tri_inverse_bf16"] += 1
        Z = torch.from_numpy(np.linalg.inv(_np(R))).float()
        return Z, Z.bfloat16(), Z.t().contiguous().bfloat16()

    def cond_estimate(self, R, Z):
        """kappa_2(R) (exact, by SVD) as a float[1] tensor."""
        self.calls["cond_estimate"] += 1
        return torch.tensor([float(np.linalg.cond(_np(R)))], dtype=torch.float32)

    def precondition_apply_bf16(self, grad, ZX2, ZG2):
        self.calls["precondition_apply_bf16"] += 1
        zx, zg = _np(ZX2[0]), _np(ZG2[0])
        return torch.from_numpy(zg @ (zg.T @ _np(grad)) @ zx @ zx.T).float()

    def inverse_split_copies(self, Z):
        """RNE bf16 halves (Z_hi, Z_lo, Z^T_hi, Z^T_lo), as ifk_inverse_split_copies."""
        self.calls["inverse_split_copies"] += 1
        Z = Z.float()
        hi = Z.bfloat16()
        lo = (Z - hi.float()).bfloat16()
        return hi, lo, hi.t().contiguous(), lo.t().contiguous()

    def precondition_apply_x3(self, grad, ZX4, ZG4):
        self.calls["precondition_apply_x3"] += 1
        zx = _np(ZX4[0]) + _np(ZX4[1])
        zg = _np(ZG4[0]) + _np(ZG4[1])
        return torch.from_numpy(zg @ (zg.T @ _np(grad)) @ zx @ zx.T).float()

    def factor_evd(self, R):
        self.calls["factor_evd"] += 1
        V, d = O.factor_evd(_np(R))
        return (torch.from_numpy(V).float(), torch.from_numpy(d).float(),
                torch.tensor([1], dtype=torch.int32))

    def laplace_scales(self, d, sqrt_n, sqrt_lam):
        self.calls["laplace_scales"] += 1
        return torch.from_numpy(1.0 / np.sqrt(sqrt_n * _np(d) + sqrt_lam)).float()

    def laplace_sample_(self, W_map, W, U_G, s_G, U_A, s_A, Xi):
        self.calls["laplace_sample"] += 1
        out = O.laplace_sample(_np(W_map), _np(U_A), _np(s_A), _np(U_G), _np(s_G), _np(Xi))
        W.copy_(torch.from_numpy(out).float())

    def gram_accumulate_(self, S, X, beta):
        self.calls["gram_accumulate"] += 1
        x = _np(X)
        prev = _np(S) if beta != 0.0 else 0.0
        S.copy_(torch.from_numpy(beta * prev + x.T @ x).float())

    def axpby(self, alpha, X, beta, Y=None):
        self.calls["axpby"] += 1
        out = alpha * _np(X) + (beta * _np(Y) if Y is not None and beta != 0.0 else 0.0)
        out = torch.from_numpy(np.asarray(out)).float()
        if Y is None:
            return out
        Y.copy_(out)
        return Y

    def gemm(self, A, B, trans_a=False, trans_b=False, math=0, alpha=1.0, beta=0.0, C=None,
             tri_a=0, tri_b=0):
        self.calls["gemm"] += 1
        a = _np(A).T if trans_a else _np(A)
        b = _np(B).T if trans_b else _np(B)
        out = alpha * (a @ b) + (beta * _np(C) if C is not None and beta != 0.0 else 0.0)
        return torch.from_numpy(np.asarray(out)).float()

    def inv_spd_damped(self, A, damping):
        self.calls["inv_spd_damped"] += 1
        return torch.from_numpy(O.classic_inverse(_np(A), damping)).float()

    def classic_precondition(self, grad, A_inv, G_inv):
        self.calls["classic_precondition"] += 1
        return torch.from_numpy(O.classic_nat(_np(grad), _np(A_inv), _np(G_inv))).float()

    def trsm(self, R, B, upper, out_dtype, math):
        self.calls["trsm"] += 1
        r = np.triu(_np(R)) if upper else np.tril(_np(R))
        return torch.from_numpy(sla.solve_triangular(r, _np(B), lower=not upper)).to(out_dtype)

    def precondition(self, grad, R_X, R_G, math):
        self.calls["precondition"] += 1
        return torch.from_numpy(O.apply_vered(_np(grad), _np(R_X), _np(R_G))).float()

    def precondition_apply(self, grad, Z_X, Z_G, math):
        self.calls["precondition_apply"] += 1
        g, zx, zg = _np(grad), _np(Z_X), _np(Z_G)
        return torch.from_numpy(zg @ (zg.T @ g) @ zx @ zx.T).float()

    def precondition_bias(self, g, Z_G):
        self.calls["precondition_bias"] += 1
        zg = _np(Z_G)
        return torch.from_numpy(zg @ (zg.T @ _np(g).reshape(-1))).float()

    def momentum_update_(self, nat, buf, W, lr, momentum, weight_decay, buf_init):
        self.calls["momentum_update"] += 1
        b = None if (buf is None or buf_init) else buf.detach().cpu().numpy()
        Wn, bn = O.momentum_step(nat.detach().reshape(W.shape).cpu().float().numpy(), b,
                                 W.detach().cpu().numpy(), lr, momentum, weight_decay)
        W.copy_(torch.from_numpy(Wn))
        if buf is not None and bn is not None:
            buf.copy_(torch.from_numpy(bn))
