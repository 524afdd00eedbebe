"""The benchmark configurations at full size on the GPU, through the exact
chains IFKFAC runs.

Linear 4096 <-> 11008 at p = 16384 (bf16): for kappa(X) in {1e1, 1e2, 1e3},
literal (singular values log-spaced in [1/kappa, 1], damping 1e-2, where the
damping dominates X^T X / p) and kappa-exposed (X scaled by sqrt(p) and
damping 0.1 / kappa^2, so kappa(R_damped) ~ kappa), both orientations, the
factor update IFKFAC times: fold_finalize by the Gram matrix + blocked
Cholesky (the panel path for a side whose status is 2) -> tri_inverse_bf16 ->
the bf16 apply, and the chain IFKFAC runs where both sides take the Gram
route: the factor with its inverse from ifk_fold_finalize_gram_inverse ->
the bf16 apply, held to the same bounds.
Bounds, each on its own part of the error:
  factor    ||R^T R - (X^T X / p + lam I)||_F / ||.||_F <= 4 kappa(R) eps_bf16
            (vacuous) and <= 5e-3 (measured at most 2.2e-3): the bf16 rounding
            of the stored factor;
  solves    against fp64 solves with the same stored factors: <= 2e-2 in bf16
            arithmetic (measured at most 1.4e-2 at kappa(R) ~ 950), <= 1e-5 in
            fp32 arithmetic (the reference's regime, triangular.py:607-628;
            measured at most 5.6e-6, as rocBLAS's fp32 trsm on the same
            factors);
  against the reference's own bf16-mode result on the same bf16 inputs
            (its factors: the exact R of [X / sqrt(p); sqrt(lam) I], RNE bf16;
            then its fp32 solves, triangular.py:607-628): <= 2e-2 where the
            damping dominates; kappa-exposed, reported;
  end to end against the fp64 closed form (G + lam I)^-1 grad (A + lam I)^-1:
            <= 2e-2 where the damping dominates; kappa-exposed, where the bf16
            storage of R alone costs the reference's own regime about
            kappa(R) 2^-9 (measured 1.5e-2 at kappa 1e2), within 2e-2 of the
            reference's own distance and of the reference regime's error on
            the same factors.
The fp64 checkers (Gram, Cholesky, solves) run in torch on the GPU.
"""
import math

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS_BF16 = 7.8125e-03
EPS32 = 1.1920929e-07


def kappa_matrix(p, n, kappa, seed):
    """p x n fp64 U diag(s) V^T on the GPU: Haar-like U, V (CholeskyQR2 of Gaussian
    matrices), s log-spaced from 1 to 1/kappa."""
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


def rel(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def damped_gram(T, lam):
    n = T.shape[1]
    return (T.double().t() @ T.double()) / T.shape[0] + lam * torch.eye(n, device=DEV,
                                                                          dtype=torch.float64)


def factor_update(hip, T, lam, out_dtype=torch.bfloat16, math_=1):
    """RawActivationHooks' consuming factor update for one side: the Gram matrix +
    blocked Cholesky in bf16 arithmetic (CholeskyQR2 blocks in fp32), the panel
    path in fp32 arithmetic if that reports status 2."""
    p = T.shape[0]
    F_, st = hip.fold_finalize(None, 0, T, 1 / math.sqrt(p), lam, out_dtype, math_,
                               cqr=math_ == 0, gram=math_ == 1)
    first = int(st.item())
    if first == 2:
        F_, st = hip.fold_finalize(None, 0, T, 1 / math.sqrt(p), lam, out_dtype, 0, cqr=False)
    return F_, first, int(st.item())


def fp64_natgrad(grad, A, G):
    """(G)^-1 grad (A)^-1 for SPD A, G (fp64, by Cholesky)."""
    LA, LG = torch.linalg.cholesky(A), torch.linalg.cholesky(G)
    return torch.cholesky_solve(torch.cholesky_solve(grad.double(), LG).t(), LA).t()


def stored_natgrad(grad, RX, RG):
    """(R_G^T R_G)^-1 grad (R_X^T R_X)^-1 in fp64 from the stored factors."""
    RX, RG = RX.double(), RG.double()
    return torch.cholesky_solve(torch.cholesky_solve(grad.double(), RG.t()).t(), RX.t()).t()


def ref_regime_natgrad(grad, RX, RG):
    """The reference's bf16-mode solves: fp32 trsm on the up-cast factors
    (triangular.py:621-628), here rocBLAS through torch, as a checker."""
    RXf, RGf = RX.float(), RG.float()
    T1 = torch.linalg.solve_triangular(RGf.t(), grad, upper=False)
    T2 = torch.linalg.solve_triangular(RGf, T1, upper=True)
    T3 = torch.linalg.solve_triangular(RXf.t(), T2.t(), upper=False)
    return torch.linalg.solve_triangular(RXf, T3, upper=True).t()


def ref_regime_factor(M):
    """The reference's bf16-mode factor of the damped Gram M: the upper factor
    with positive diagonal of [X / sqrt(p); sqrt(lam) I] (the R of its
    Householder QR, triangular.py:284,299-301,411-416, here by the fp64
    Cholesky of M, which gives the same R to about kappa^2 1e-16), then its
    RNE bf16 cast (ifkfac.py:292-294)."""
    return torch.linalg.cholesky(M).t().contiguous().bfloat16()


def kappa_of_gram(M):
    """kappa of the factor R of an SPD M = R^T R: sqrt of M's eigenvalue ratio."""
    w = torch.linalg.eigvalsh(M)
    return math.sqrt((w[-1] / w[0]).item())


@pytest.mark.parametrize("n_in,n_out", [(4096, 11008), (11008, 4096)])
@pytest.mark.parametrize("kappa", [1e1, 1e2, 1e3])
@pytest.mark.parametrize("exposed", [False, True])
def test_linear_4096_11008_kappa_sweep_timed_chain(hip, n_in, n_out, kappa, exposed):
    p = 16384
    X = kappa_matrix(p, n_in, kappa, 1)
    D = kappa_matrix(p, n_out, 1e1, 2)
    if exposed:
        X, D = X * math.sqrt(p), D * math.sqrt(p)
        lam = 0.1 / kappa ** 2
    else:
        lam = 1e-2
    Xb, Db = X.bfloat16(), D.bfloat16()
    del X, D
    A, G = damped_gram(Xb, lam), damped_gram(Db, lam)
    FX, sx0, sx = factor_update(hip, Xb, lam)
    FG, sg0, sg = factor_update(hip, Db, lam)
    assert sx == 1 and sg == 1
    # kappa(R_X) of the construction (about 1 where the damping dominates)
    kX = math.sqrt((1 + lam) / (1 / kappa ** 2 + lam)) if exposed else 1.0
    for Fm, M in ((FX, A), (FG, G)):
        e = rel(Fm.double().t() @ Fm.double(), M)
        assert e <= 5e-3, e        # hence also <= 4 kappa eps_bf16 (kappa >= 1)
        d = torch.diagonal(Fm)
        assert bool((d > 0).all()) and torch.count_nonzero(torch.tril(Fm, -1)).item() == 0
    grad = torch.randn(n_out, n_in, device=DEV,
                       generator=torch.Generator(device=DEV).manual_seed(3)) * 0.1
    ZX, ZG = hip.tri_inverse_bf16(FX), hip.tri_inverse_bf16(FG)
    nat = hip.precondition_apply_bf16(grad, (ZX[1], ZX[2]), (ZG[1], ZG[2]))
    stored = stored_natgrad(grad, FX, FG)
    e_solve = rel(nat, stored)
    nat32 = hip.precondition_apply(grad, hip.tri_inverse(FX, 0), hip.tri_inverse(FG, 0), 0)
    e_solve32 = rel(nat32, stored)
    truth = fp64_natgrad(grad, A, G)
    ref = ref_regime_natgrad(grad, FX, FG)
    e_truth, e_ref = rel(nat, truth), rel(ref, truth)
    # the reference's own bf16-mode result on the same bf16 inputs: its factors
    # (exact R, RNE bf16), then its fp32 solves
    ref_own = ref_regime_natgrad(grad, ref_regime_factor(A), ref_regime_factor(G))
    e_own, e_own_truth = rel(nat, ref_own), rel(ref_own, truth)
    # the apply IFKFAC takes for a layer with a factor of kappa above
    # KAPPA_BF16_MAX: fp32-accurate solves from the split inverse copies
    nat3 = hip.precondition_apply_x3(grad, hip.inverse_split_copies(ZX[0]),
                                     hip.inverse_split_copies(ZG[0]))
    e3_own, e3_truth = rel(nat3, ref_own), rel(nat3, truth)
    print(f"kappa(R_X)={kX:.1f} status=({sx0},{sg0}) solve bf16 {e_solve:.2e} fp32 {e_solve32:.2e}"
          f" | vs the reference's bf16-mode result: bf16 apply {e_own:.2e}, fp32 apply "
          f"{e3_own:.2e} | vs closed form: ours {e_truth:.2e} / {e3_truth:.2e}, reference "
          f"{e_own_truth:.2e}, reference solves on our factors {e_ref:.2e}")
    assert e_solve <= 2e-2
    assert e_solve32 <= 1e-5
    if not exposed:
        assert e_own <= 2e-2 and e3_own <= 2e-2
        assert e_truth <= 2e-2
    else:
        # kappa(R_X) up to 1e3: the bf16 storage of R moves both results from
        # the closed form, each its own way; reported, and ours held to the
        # reference's own distance from the closed form
        assert e_truth <= e_own_truth + 2e-2 and e3_truth <= e_own_truth + 2e-2
        assert e_truth <= e_ref + 2e-2
    if sx0 == 1 and sg0 == 1:
        # the factor and its inverse from one call, as IFKFAC takes them
        inv = []
        for T, Fm in ((Xb, FX), (Db, FG)):
            out, st, _, (Z, Zb, ZT) = hip.fold_finalize_gram_batched(
                None, 0, [T], 1 / math.sqrt(p), lam, torch.bfloat16, with_inverse=True)
            assert st.item() == 1 and torch.equal(out[0], Fm)
            inv.append((Zb[0], ZT[0]))
        nat_f = hip.precondition_apply_bf16(grad, inv[0], inv[1])
        e_fs, e_ft = rel(nat_f, stored), rel(nat_f, truth)
        print(f"  with the inverse from the factor call: solve {e_fs:.2e}, vs closed form {e_ft:.2e}")
        assert e_fs <= 2e-2
        assert e_ft <= (2e-2 if not exposed else e_ref + 2e-2)


@pytest.mark.parametrize("side", ["X", "G"])
def test_linear_4096_11008_flagged_block_takes_the_panel_path(hip, side):
    """A side whose Cholesky pivot test fails at full size (two equal columns of
    large scale: the Gram's pivot falls to the damping, 1e-6 of its diagonal)
    reports status 2, and the panel path (ifk_fold_finalize) gives the
    factor, which then runs through the bf16 inverse and apply: factor and
    solves within the bounds of the sweep."""
    p, n_in, n_out, lam = 16384, 4096, 11008, 1e-2
    g = torch.Generator(device=DEV).manual_seed(21)
    X = (torch.randn(p, n_in, device=DEV, generator=g) * 0.01).to(torch.float64)
    D = (torch.randn(p, n_out, device=DEV, generator=g) * 0.01).to(torch.float64)
    T = X if side == "X" else D
    j = T.shape[1] // 2 + 7
    T[:, j] = torch.randn(p, device=DEV, generator=g, dtype=torch.float64) * 80.0
    T[:, j + 300] = T[:, j]
    Xb, Db = X.bfloat16(), D.bfloat16()
    FX, sx0, sx = factor_update(hip, Xb, lam)
    FG, sg0, sg = factor_update(hip, Db, lam)
    assert (sx0 if side == "X" else sg0) == 2
    assert sx == 1 and sg == 1
    for Fm, Tb in ((FX, Xb), (FG, Db)):
        M = damped_gram(Tb, lam)
        assert rel(Fm.double().t() @ Fm.double(), M) <= 5e-3
    grad = torch.randn(n_out, n_in, device=DEV, generator=g) * 0.1
    ZX, ZG = hip.tri_inverse_bf16(FX), hip.tri_inverse_bf16(FG)
    nat = hip.precondition_apply_bf16(grad, (ZX[1], ZX[2]), (ZG[1], ZG[2]))
    assert rel(nat, stored_natgrad(grad, FX, FG)) <= 2e-2


def _capture(model):
    acts, grads, hs = {}, {}, []
    for m in model.modules():
        if isinstance(m, nn.Linear):
            hs.append(m.register_forward_hook(
                lambda mod, i, o: acts.__setitem__(mod, i[0].detach().clone())))
            hs.append(m.register_full_backward_hook(
                lambda mod, gi, go: grads.__setitem__(mod, go[0].detach().clone())))
    return acts, grads, hs


def test_mlp_4x4096_gelu_ifkfac_step_bf16(hip):
    """4 x (Linear(4096, 4096) + GELU), p = 8192 tokens with kappa(X) = 1e2 input,
    IFKFAC(use_true_bf16=True, factor_update_freq=1, momentum=0.9).step(): all
    four layers go through one same-shape bucket; each layer's solves run in bf16
    arithmetic when the Gram path's upper bound of kappa_2 of both its factors
    is at most 1.5, and in fp32 otherwise
    (the first layer's input is near-isotropic after damping, the GELU inputs
    of layers 2-4 are not); every layer's bf16 factors
    against its captured activations and deltas (the sweep's Gram bound); each
    layer's natural gradient (its momentum buffer after the first step) against
    fp64 solves with its stored factors at 2e-2, against the reference's own
    bf16-mode result on the same captured rows (exact factors, RNE bf16, fp32
    solves) at 2e-2, and against the fp64 closed form within 2e-2 of the
    reference regime's error on the same factors (the
    GELU inputs of layers 2-4 carry a mean component, so their kappa(R) is far
    above the damping-dominated 1 and the bf16 storage of R shows)."""
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    p, n, lam = 8192, 4096, 1e-2
    layers = [nn.Linear(n, n) for _ in range(4)]
    model = nn.Sequential(*[m for l in layers for m in (l, nn.GELU())]).to(DEV)
    opt = IFKFAC(model, lr=1e-3, damping=lam, factor_update_freq=1, momentum=0.9,
                 use_true_bf16=True)
    x = kappa_matrix(p, n, 1e2, 5).float()
    target = torch.randn(p, n, device=DEV, generator=torch.Generator(device=DEV).manual_seed(6))
    acts, grads, hs = _capture(model)
    loss = ((model(x) - target) ** 2).mean()
    loss.backward()
    for h in hs:
        h.remove()
    gW = {l: l.weight.grad.detach().clone() for l in layers}
    import contextlib, io
    with contextlib.redirect_stdout(io.StringIO()):
        opt.step()
    torch.cuda.synchronize()
    assert set(opt._factors) == set(layers)
    from ifkfac_amd.ifkfac import KAPPA_BF16_MAX
    for l in layers:
        RX, RG = opt._factors[l]
        kx, kg = opt._kappas[l]
        bf16_solves = max(kx, kg) <= KAPPA_BF16_MAX
        assert (l in opt._inverse_copies) == bf16_solves
        kx_true = kappa_of_gram(RX.double().t() @ RX.double())
        # the Gram path's bound sqrt(1 + ||X^T X / p||_F / lam) bounds kappa_2 of
        # the exact factor; the bf16 rounding of the stored one moves its kappa by
        # up to about 2^-8 relative (measured 0.17 % above a tight bound: the
        # GELU inputs' Gram matrix is dominated by one mean direction)
        assert kx >= 0.99 * kx_true
        assert RX.dtype == torch.bfloat16 and RG.dtype == torch.bfloat16
        A, G = damped_gram(acts[l], lam), damped_gram(grads[l], lam)
        for Fm, M in ((RX, A), (RG, G)):
            assert rel(Fm.double().t() @ Fm.double(), M) <= 5e-3
        nat = opt._momentum_buffers[l]
        e_solve = rel(nat, stored_natgrad(gW[l], RX, RG))
        truth = fp64_natgrad(gW[l], A, G)
        e_truth = rel(nat, truth)
        e_ref = rel(ref_regime_natgrad(gW[l], RX, RG), truth)
        ref_own = ref_regime_natgrad(gW[l], ref_regime_factor(A), ref_regime_factor(G))
        e_own, e_own_truth = rel(nat, ref_own), rel(ref_own, truth)
        print(f"kappa(R_X) {kx:.2f} kappa(R_G) {kg:.2f} ({'bf16' if bf16_solves else 'fp32'}"
              f" solves): solve {e_solve:.2e}; vs the reference's bf16-mode result "
              f"{e_own:.2e}; vs closed form ours {e_truth:.2e}, reference {e_own_truth:.2e}")
        assert e_solve <= 2e-2
        assert e_own <= 2e-2
        assert e_truth <= e_ref + 2e-2


@pytest.mark.parametrize("n", [4096, 11008])
@pytest.mark.parametrize("kappa", [1e1, 1e2, 1e3])
def test_cholesky_leg_kappa_sweep(hip, n, kappa):
    """The Cholesky leg of the 4096 / 11008 configuration (bf16_linalg.py:247-280,
    the Gram factors the Classic control forms): A = X^T X / p + lam I at
    p = 16384 with X scaled by sqrt(p) (eig(X^T X / p) = s^2, log-spaced in
    [1 / kappa^2, 1]) and the configuration's damping lam = 1e-2, so kappa(A)
    is 50 to 100 over the sweep and the bf16-rounded A_b stays positive definite
    (with damping 0.1 / kappa^2 instead, A_b is indefinite from kappa = 1e2 on:
    the 1e-7 pivot clamp of the reference's rule then lets the factor grow
    without bound, in the reference as here -- the kappa^2 the Gram route
    avoids; the clamp itself is pinned against the oracle on small indefinite
    input in test_gpu_parity.py).
      cholesky_bf16 (ifk_potrf): ||L L^T - A_b||_F / ||A_b||_F at most twice the
        same error of the reference regime's factor (fp32 Cholesky of A_b,
        stored as bf16), plus 1e-3;
      inv_spd_bf16 (ifk_inv_spd): against the fp64 inverse of A_b at the
        bf16-mode 2e-2 (bf16 arithmetic in each stage, as the reference's
        bf16 solves; the fp32 Cholesky inverse rounded once to bf16 is printed
        beside it);
      inv_spd_damped (fp32, the Classic control's inverse): (X^T X / p + lam I)^-1
        within 8 sqrt(n) kappa(A) eps32 of fp64."""
    p, lam = 16384, 1e-2
    Xb = (kappa_matrix(p, n, kappa, 9) * math.sqrt(p)).bfloat16()
    Au = (Xb.double().t() @ Xb.double()) / p
    eye = torch.eye(n, device=DEV, dtype=torch.float64)
    A = Au + lam * eye
    Ab = A.to(torch.bfloat16)
    Ab64 = Ab.double()
    L = hip.potrf(Ab, torch.bfloat16, 1)
    assert bool(torch.isfinite(L.float()).all())
    assert torch.count_nonzero(torch.triu(L, 1)).item() == 0
    assert bool((torch.diagonal(L).float() > 0).all())
    L32, info = torch.linalg.cholesky_ex(Ab.float())
    assert int(info.item()) == 0
    nA = Ab64.norm()
    e_l = ((L.double() @ L.double().t() - Ab64).norm() / nA).item()
    Lr = L32.bfloat16().double()
    e_lr = ((Lr @ Lr.t() - Ab64).norm() / nA).item()
    Xi = hip.inv_spd(Ab, torch.bfloat16, 1)
    inv64 = torch.cholesky_inverse(torch.linalg.cholesky(Ab64))
    e_i = ((Xi.double() - inv64).norm() / inv64.norm()).item()
    e_ir = ((torch.cholesky_inverse(L32).bfloat16().double() - inv64).norm() /
            inv64.norm()).item()
    w = torch.linalg.eigvalsh(A)
    kap = (w[-1] / w[0]).item()
    print(f"n={n} kappa={kappa:g} (kappa(A) {kap:.3g}): cholesky_bf16 {e_l:.2e} (reference "
          f"regime {e_lr:.2e}); inv_spd_bf16 {e_i:.2e} (fp32 inverse rounded once {e_ir:.2e})")
    assert e_l <= 2 * e_lr + 1e-3
    assert e_i <= 2e-2
    Xd = hip.inv_spd_damped(Au.float(), lam)
    inv_d = torch.cholesky_inverse(torch.linalg.cholesky(A))
    e_d = ((Xd.double() - inv_d).norm() / inv_d.norm()).item()
    print(f"  inv_spd_damped {e_d:.2e} (bound {8 * math.sqrt(n) * kap * EPS32:.2e})")
    assert e_d <= 8 * math.sqrt(n) * kap * EPS32
