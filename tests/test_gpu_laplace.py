"""The Laplace consumer on the GPU through the C ABI: the factor EVD
(ifk_factor_evd, one-sided block Jacobi SVD of R) and the posterior sample
(ifk_laplace_scales, ifk_laplace_sample).

Bounds:
  EVD       every eigenvalue of R^T R to relative 2e-5 of itself against
            numpy's SVD of the same fp32 R (one-sided Jacobi keeps the small
            singular values' relative accuracy; the formed R^T R would lose
            them at kappa(R)^2 eps); ||V^T V - I||_max <= 1e-4;
            ||V diag(d) V^T - R^T R||_F / ||R^T R||_F <= 1e-5; d descending;
            converged (sweeps > 0); the lower triangle of R never read.
  sample    W_map + U_G diag(s_G) Xi diag(s_A) U_A^T on the same Xi: <= 1e-5 of
            the perturbation's scale (fp32 products); the scales to 2 ulp.
"""
import math
import time

import numpy as np
import pytest
import torch

from oracle import ifk_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _factor(p, n, kappa, seed, lam=1e-3):
    rng = np.random.default_rng(seed)
    X = O.kappa_matrix(p, n, kappa, rng) * math.sqrt(p)
    return O.get_factor(O.streaming_tsqr_update(None, X), p, lam).astype(np.float32)


@pytest.mark.parametrize("n,kappa", [(1, 1.0), (17, 10.0), (100, 1e2), (300, 1e3), (768, 1e2),
                                     (1100, 1e2)])
def test_factor_evd(hip, n, kappa):
    R = _factor(max(2 * n, 4), n, kappa, n)
    Rt = torch.tensor(R, device=DEV)
    Rt_junk = Rt + torch.tril(torch.full_like(Rt, 7.0), -1)   # lower triangle must not matter
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    V, d, sweeps = hip.factor_evd(Rt_junk)
    torch.cuda.synchronize()
    ms = 1e3 * (time.perf_counter() - t0)
    s = np.linalg.svd(R.astype(np.float64), compute_uv=False)
    dn = d.double().cpu().numpy()
    Vn = V.double().cpu().numpy()
    rel = np.abs(dn - s * s) / (s * s)
    print(f"factor_evd n={n} kappa(R)={s[0] / s[-1]:.3g}: {ms:.1f} ms, sweeps {sweeps.item()}, "
          f"max eig rel {rel.max():.2e}")
    assert sweeps.item() > 0
    assert rel.max() <= 2e-5
    assert np.all(np.diff(dn) <= 0)
    assert np.abs(Vn.T @ Vn - np.eye(n)).max() <= 1e-4
    A = R.astype(np.float64).T @ R.astype(np.float64)
    assert np.linalg.norm(Vn @ np.diag(dn) @ Vn.T - A) / np.linalg.norm(A) <= 1e-5


@pytest.mark.parametrize("n", [2304, 3072])
def test_factor_evd_vit_widths(hip, n):
    """The widths of the ViT-B capture's layers (768 -> 2304, 768 -> 3072)."""
    R = _factor(2 * n, n, 1e2, 5)
    V, d, sweeps = hip.factor_evd(torch.tensor(R, device=DEV))
    s = np.linalg.svd(R.astype(np.float64), compute_uv=False)
    rel = np.abs(d.double().cpu().numpy() - s * s) / (s * s)
    Vn = V.double().cpu().numpy()
    print(f"factor_evd n={n}: sweeps {sweeps.item()}, max eig rel {rel.max():.2e}")
    assert sweeps.item() > 0 and rel.max() <= 2e-5
    assert np.abs(Vn.T @ Vn - np.eye(n)).max() <= 1e-4


@pytest.mark.parametrize("n_out,n_in", [(10, 256), (256, 128), (768, 768)])
def test_laplace_sample(hip, n_out, n_in):
    rng = np.random.default_rng(n_out + n_in)
    U_A = np.linalg.qr(rng.standard_normal((n_in, n_in)))[0].astype(np.float32)
    U_G = np.linalg.qr(rng.standard_normal((n_out, n_out)))[0].astype(np.float32)
    d_A = np.sort(rng.uniform(1e-4, 2.0, n_in))[::-1].astype(np.float32)
    d_G = np.sort(rng.uniform(1e-4, 2.0, n_out))[::-1].astype(np.float32)
    W0 = rng.standard_normal((n_out, n_in)).astype(np.float32)
    Xi = rng.standard_normal((n_out, n_in)).astype(np.float32)
    sA = hip.laplace_scales(torch.tensor(d_A, device=DEV), math.sqrt(5000.0), math.sqrt(10.0))
    sG = hip.laplace_scales(torch.tensor(d_G, device=DEV), math.sqrt(5000.0), math.sqrt(10.0))
    wA = O.laplace_scales(d_A, 5000, 10.0)
    assert np.allclose(sA.double().cpu().numpy(), wA, rtol=2.4e-7)
    W = torch.empty(n_out, n_in, device=DEV)
    hip.laplace_sample_(torch.tensor(W0, device=DEV), W, torch.tensor(U_G, device=DEV), sG,
                        torch.tensor(U_A, device=DEV), sA, torch.tensor(Xi, device=DEV))
    want = O.laplace_sample(W0, U_A, sA.double().cpu().numpy(), U_G, sG.double().cpu().numpy(),
                            Xi)
    dW = want - W0
    assert np.abs(W.double().cpu().numpy() - want).max() <= 1e-5 * np.abs(dW).max() + 1e-6


def test_laplace_posterior_end_to_end(hip):
    """IFKFAC capture -> get_factors -> factors_to_evd -> LaplacePosterior on the
    GPU: the draws equal the restated sample on the same generator's Xi."""
    import torch.nn as nn
    from ifkfac_amd import IFKFAC, LaplacePosterior, factors_to_evd
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(128, 256), nn.ReLU(), nn.Linear(256, 10)).to(DEV)
    opt = IFKFAC(model, lr=0.0, damping=1e-3, factor_update_freq=1000)
    g = torch.Generator(device=DEV).manual_seed(0)
    for _ in range(3):
        x = torch.randn(512, 128, device=DEV, generator=g)
        logits = model(x)
        y = torch.multinomial(torch.softmax(logits.float(), -1), 1, generator=g).squeeze(-1)
        model.zero_grad(set_to_none=True)
        torch.nn.functional.cross_entropy(logits, y).backward()
    factors = opt.hooks.get_factors()
    opt.hooks.remove()
    evd = factors_to_evd(factors)
    W0 = {m: m.weight.detach().clone() for m in factors}
    post = LaplacePosterior(model, evd, prior_precision=10.0, dataset_size=5000)
    post.sample_in_place(generator=torch.Generator(device=DEV).manual_seed(3))
    gg = torch.Generator(device=DEV).manual_seed(3)
    for m in factors:
        U_A, d_A, U_G, d_G = evd[m]
        xi = torch.randn(U_G.shape[0], U_A.shape[0], device=DEV, generator=gg)
        sA = O.laplace_scales(d_A.double().cpu().numpy(), 5000, 10.0)
        sG = O.laplace_scales(d_G.double().cpu().numpy(), 5000, 10.0)
        want = O.laplace_sample(W0[m].double().cpu().numpy(), U_A.double().cpu().numpy(), sA,
                                U_G.double().cpu().numpy(), sG, xi.double().cpu().numpy())
        dW = want - W0[m].double().cpu().numpy()
        got = m.weight.detach().double().cpu().numpy()
        assert np.abs(got - want).max() <= 1e-5 * np.abs(dW).max() + 1e-6
    post.restore_map()
    for m in factors:
        assert torch.equal(m.weight.detach(), W0[m])
