"""The Classic K-FAC control on the GPU, through the C ABI: the Gram sums of
KFACHooks (ifk_gram_accumulate), the damped inverses of ClassicKFAC
(ifk_inv_spd_damped), its natural gradient (ifk_classic_precondition) and a
ClassicKFAC run against the same host code on the oracle backend.

Bounds:
  Gram sums     fp32 input in fp32 arithmetic: ||S - X^T X||_F / ||X^T X||_F
                <= 1e-5 (fp32 accumulation over p rows); bf16 input: exact
                products of the bf16 values with fp32 accumulation, the same
                bound against the fp64 Gram of the bf16 values; S exactly
                symmetric.
  inverses      ||X - (A + lam I)^{-1}||_F / ||.||_F <= 8 sqrt(n) kappa eps32, the
                forward error of a backward-stable Cholesky inverse
                (kappa = kappa_2(A + lam I)); at the configuration's full sizes
                (n = 4096 and 11008, A = X^T X / p + lam I) as well.
  natural grad  G^{-1} g A^{-1} from the fp32 inverses: <= 1e-5 against fp64
                products of the same inverses.
  the contrast  at kappa(X) = 1e2 with X scaled by sqrt(p) (kappa-exposed,
                damping 1e-5), the Classic natural gradient (fp32 Gram, fp32
                inverse) against the fp64 closed form loses the small
                eigenvalues of the formed Gram; the factor path (fp32 fold,
                fp32 solves) keeps them: at least 5 times smaller error (the
                reference's own stability contrast, tests/test_bf16_stability.py,
                asks ratio >= 5).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import ifk_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS32 = 1.1920929e-07


def _rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def _kappa_matrix(p, n, kappa, seed):
    """p x n fp64 U diag(s) V^T on the GPU, s log-spaced from 1 to 1/kappa."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    k = min(p, n)

    def orth(m):
        Q = torch.randn(m, k, device=DEV, dtype=torch.float64, generator=g)
        for _ in range(2):
            L = torch.linalg.cholesky(Q.t() @ Q)
            Q = torch.linalg.solve_triangular(L, Q.t(), upper=False).t()
        return Q

    U, V = orth(p), orth(n)
    s = torch.logspace(0, -math.log10(kappa), k, device=DEV, dtype=torch.float64)
    return (U * s) @ V.t()


@pytest.mark.parametrize("p,n", [(300, 128), (3000, 700), (2048, 1100), (8192, 4096)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_gram_accumulate(hip, p, n, xdt):
    g = torch.Generator(device=DEV).manual_seed(p + n)
    X1 = torch.randn(p, n, device=DEV, generator=g).to(xdt)
    X2 = (torch.randn(p // 2 + 1, n, device=DEV, generator=g) + 0.5).to(xdt)
    S = torch.full((n, n), float("nan"), device=DEV)     # beta = 0 never reads S
    hip.gram_accumulate_(S, X1, 0.0)
    want = X1.double().t() @ X1.double()
    assert _rel(S, want) <= 1e-5
    assert torch.equal(S, S.t())
    hip.gram_accumulate_(S, X2, 1.0)
    want = want + X2.double().t() @ X2.double()
    assert _rel(S, want) <= 1e-5
    assert torch.equal(S, S.t())
    # the average of the two windows' rows, as get_factors forms it
    A = hip.axpby(1.0 / (X1.shape[0] + X2.shape[0]), S, 0.0)
    assert torch.equal(A, S * (1.0 / (X1.shape[0] + X2.shape[0])))


@pytest.mark.parametrize("n,kappa_x,lam", [(64, 10.0, 1e-2), (300, 1e2, 1e-3), (1100, 1e2, 1e-4),
                                           (2100, 30.0, 1e-3)])
def test_inv_spd_damped(hip, n, kappa_x, lam):
    X = _kappa_matrix(2 * n, n, kappa_x, n) * math.sqrt(2 * n)
    A = (X.t() @ X / (2 * n)).float()
    Ad = A.double() + lam * torch.eye(n, device=DEV, dtype=torch.float64)
    want = torch.linalg.inv(Ad)
    got = hip.inv_spd_damped(A, lam)
    kap = (1.0 + lam) / (kappa_x ** -2 + lam)     # eig(X^T X / p) = s^2 by construction
    e = _rel(got, want)
    print(f"inv_spd_damped n={n}: rel {e:.3e}, kappa {kap:.3g}")
    assert e <= 8 * math.sqrt(n) * kap * EPS32


@pytest.mark.parametrize("n", [4096, 11008])
def test_inv_spd_damped_full_size(hip, n):
    """The Classic leg of the 4096 <-> 11008, p = 16384 configuration: the damped
    inverse of X^T X / p + lam I at the layer's full width."""
    p, lam = 16384, 1e-2
    X = _kappa_matrix(p, n, 1e2, 7) * math.sqrt(p)
    A = (X.t() @ X / p).float()
    del X
    Ad = A.double() + lam * torch.eye(n, device=DEV, dtype=torch.float64)
    want = torch.linalg.inv(Ad)
    got = hip.inv_spd_damped(A, lam)
    kap = (1.0 + lam) / (1e-4 + lam)
    e = _rel(got, want)
    print(f"inv_spd_damped n={n}: rel {e:.3e}, kappa {kap:.3g}")
    assert e <= 8 * math.sqrt(n) * kap * EPS32


@pytest.mark.parametrize("n_out,n_in", [(256, 128), (1100, 700), (10, 300), (4096, 4096)])
def test_classic_precondition(hip, n_out, n_in):
    g = torch.Generator(device=DEV).manual_seed(n_out + n_in)
    Ai = torch.randn(n_in, n_in, device=DEV, generator=g) / math.sqrt(n_in)
    Gi = torch.randn(n_out, n_out, device=DEV, generator=g) / math.sqrt(n_out)
    grad = torch.randn(n_out, n_in, device=DEV, generator=g)
    got = hip.classic_precondition(grad, Ai, Gi)
    want = Gi.double() @ grad.double() @ Ai.double()
    assert _rel(got, want) <= 1e-5


def test_kappa_squared_contrast(hip):
    """kappa(X) = 1e2, kappa-exposed: the Classic natural gradient (explicit Gram,
    damped inverse) against the factor path's (R_d = chol of the same damped Gram,
    fp32 solves), both in fp32 arithmetic, against the fp64 closed form."""
    p, n, lam = 4096, 512, 1e-5
    X = _kappa_matrix(p, n, 1e2, 3) * math.sqrt(p)
    D = _kappa_matrix(p, n, 10.0, 4) * math.sqrt(p)
    g = torch.Generator(device=DEV).manual_seed(8)
    grad = torch.randn(n, n, device=DEV, generator=g, dtype=torch.float64)
    eye = torch.eye(n, device=DEV, dtype=torch.float64)
    Ad = X.t() @ X / p + lam * eye
    Gd = D.t() @ D / p + lam * eye
    want = torch.linalg.solve(Gd, torch.linalg.solve(Ad, grad.t()).t())
    # Classic: fp32 Gram sums of fp32 activations, fp32 damped inverses
    S_A = torch.empty(n, n, device=DEV)
    S_G = torch.empty(n, n, device=DEV)
    hip.gram_accumulate_(S_A, X.float(), 0.0)
    hip.gram_accumulate_(S_G, D.float(), 0.0)
    A = hip.axpby(1.0 / p, S_A, 0.0)
    G = hip.axpby(1.0 / p, S_G, 0.0)
    nat_c = hip.classic_precondition(grad.float(), hip.inv_spd_damped(A, lam),
                                     hip.inv_spd_damped(G, lam))
    # factor path: fp32 fold + finalize of the same activations, fp32 solves
    R_X, _ = hip.fold_finalize(None, 0, X.float(), 1 / math.sqrt(p), lam, torch.float32, 0)
    R_G, _ = hip.fold_finalize(None, 0, D.float(), 1 / math.sqrt(p), lam, torch.float32, 0)
    nat_f = hip.precondition(grad.float(), R_X, R_G, 0)
    e_c, e_f = _rel(nat_c, want), _rel(nat_f, want)
    print(f"kappa(X) 1e2 exposed: classic {e_c:.3e}, factor path {e_f:.3e}")
    # measured on the CPU in torch fp32 (LAPACK): 6.3e-5 against 1.5e-6
    assert 5 * e_f <= e_c


def test_classic_kfac_matches_oracle_backend(hip):
    """ClassicKFAC on the GPU and the same host code on the oracle backend (fp64
    numpy at every seam), 6 steps of the demo MLP with freq 2, momentum, decay
    and the EMA blend: the weights agree to 1e-4 of their scale (the forward and
    backward passes themselves differ by fp32 rounding between the devices)."""
    from ifkfac_amd import ClassicKFAC, _backend
    from oracle_backend import OracleBackend

    def run(device, backend):
        prev = _backend.set_backend(backend)
        try:
            torch.manual_seed(0)
            model = nn.Sequential(nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 10)).to(device)
            opt = ClassicKFAC(model, lr=1e-3, damping=1e-2, factor_update_freq=2,
                              decomp_update_freq=2, momentum=0.9, weight_decay=1e-3, gamma=0.5)
            g = torch.Generator().manual_seed(0)
            X = torch.randn(256, 128, generator=g).to(device)
            Y = torch.randint(0, 10, (256,), generator=g).to(device)
            out = []
            for _ in range(6):
                opt.zero_grad()
                torch.nn.functional.cross_entropy(model(X), Y).backward()
                opt.step()
                out.append([p.detach().double().cpu().numpy().copy() for p in model.parameters()])
            return out
        finally:
            _backend.set_backend(prev)

    gpu = run(DEV, hip)
    cpu = run("cpu", OracleBackend())
    for step, (a, b) in enumerate(zip(gpu, cpu)):
        for pa, pb in zip(a, b):
            assert np.abs(pa - pb).max() <= 1e-4 * max(1.0, np.abs(pb).max()), step
