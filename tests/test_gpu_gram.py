"""The factor update by Gram matrix + blocked Cholesky (ifk_fold_finalize_gram)
against the fp64 closed form, through the C ABI.

The path reads [R_in; X] as its RNE bf16 rounding (as every bf16-arithmetic
path does), so its closed form is chol((bf16(R_in)^T bf16(R_in) +
bf16(X)^T bf16(X)) / rows + lambda I), computed in fp64.  Bounds:
  fp32 output   ||R^T R - A||_F / ||A||_F <= 3e-5: what is left of the
                products' bf16 hi/lo splitting (about 2^-17 of |L||L^T| per
                product) and the fp32 accumulation; a forgotten lo term
                (2^-9 per entry) or a dropped Schur update fails it.
  bf16 output   exactly the RNE cast of the fp32 output.
  kappa bound   sqrt(1 + ||P^T P / rows||_F / lambda) to 1e-4 (fp64 formula on the
                same rows), and never below kappa_2 of the fp64 factor.
  status        1 for well-posed input; 2 when a pivot falls below 1e-3 of its
                Gram diagonal (rank deficiency without damping) or the input is
                not finite; the panel path then gives the factor or flag 0.
"""
import math

import numpy as np
import pytest
import torch

from oracle import ifk_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
EPS_BF16 = 7.8125e-03


def _bf16_np(t):
    return t.to(torch.bfloat16).double().cpu().numpy()


def _gram_rel(R, Ro):
    R = R.double().cpu().numpy() if isinstance(R, torch.Tensor) else R
    a = R.T @ R
    b = Ro.T @ Ro
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def _kappa(Ro):
    s = np.linalg.svd(Ro, compute_uv=False)
    return s[0] / max(s[-1], 1e-300)


def _fold_chunks(hip, chunks, n):
    R = torch.zeros(n, n, device=DEV)
    r = 0
    for X in chunks:
        r = hip.fold_(R, r, X, 0)
    return R, r


@pytest.mark.parametrize("prev,p,n,lam", [
    ([], 500, 300, 1e-2), ([300], 500, 300, 1e-2), ([64], 30, 128, 1e-2), ([], 64, 64, 1e-3),
    ([], 20, 50, 1e-1), ([], 1, 600, 1.0), ([], 4000, 1024, 1e-2), ([], 4000, 1536, 1e-2),
    ([1200], 1200, 2100, 1e-2), ([2000], 100, 1030, 1e-3), ([], 3000, 3100, 1e-2),
    ([], 5000, 4200, 1e-2), ([], 700, 5000, 1e-1),
])
def test_fold_finalize_gram_matches_closed_form(hip, prev, p, n, lam):
    """Single block (n <= 1024), two blocks (no far update), three and more (near and
    far Schur updates on two streams, part A and the rest), a running factor, fewer
    rows than columns under damping."""
    g = torch.Generator(device=DEV).manual_seed(p + n + len(prev))
    Xs = [torch.randn(q, n, device=DEV, generator=g) for q in prev]
    X = torch.randn(p, n, device=DEV, generator=g)
    R, r = _fold_chunks(hip, Xs, n)
    R_before = R.clone()
    rows = sum(prev) + p
    Rd, st = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.float32, 1, gram=True)
    assert st.item() == 1
    assert torch.equal(R, R_before)                  # the running factor is not touched
    parts = ([_bf16_np(R[:r])] if r > 0 else []) + [_bf16_np(X)]
    want = O.chol_factor(parts, rows, lam)
    e = _gram_rel(Rd, want)
    print(f"n={n} p={p} r_in={r}: gram rel {e:.3e}")
    assert e <= 3e-5
    Rg = Rd.double().cpu().numpy()
    assert np.all(np.diag(Rg) > 0) and not np.any(np.tril(Rg, -1))
    Rb, st, kb = hip.fold_finalize(R, r, X, 1 / math.sqrt(rows), lam, torch.bfloat16, 1,
                                   gram=True, with_kappa=True)
    assert st.item() == 1 and torch.equal(Rb, Rd.to(torch.bfloat16))
    # kappa bound: sqrt(1 + ||P^T P / rows||_F / lam) of the same rows, never below
    # kappa_2 of the factor
    P = np.concatenate(parts, axis=0)
    want_kb = math.sqrt(1.0 + np.linalg.norm(P.T @ P / rows) / lam)
    assert abs(kb.item() - want_kb) <= 1e-4 * want_kb
    assert kb.item() >= (1 - 1e-4) * _kappa(want)


@pytest.mark.parametrize("p,n,kappa", [(4096, 1024, 1e2), (6000, 2600, 1e1), (8192, 3072, 1e2),
                                       (2048, 700, 1e2)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_fold_finalize_gram_kappa(hip, p, n, kappa, xdt):
    """kappa-exposed input (X sqrt(p), so kappa(R_damped) ~ kappa): the factor's Gram
    error against the fp64 closed form of the bf16-rounded input stays at the level of
    the split products, far inside 4 kappa eps_bf16, and well below the bf16 panel
    path's error on the same (exact bf16) input."""
    rng = np.random.default_rng(p + n)
    X = torch.from_numpy(O.kappa_matrix(p, n, kappa, rng).astype(np.float32) * math.sqrt(p))
    X = X.to(xdt).to(DEV)
    lam = 1e-2
    want = O.chol_factor([_bf16_np(X)], p, lam)
    Rd, st = hip.fold_finalize(None, 0, X, 1 / math.sqrt(p), lam, torch.float32, 1, gram=True)
    assert st.item() == 1
    e = _gram_rel(Rd, want)
    print(f"kappa {kappa:g} n={n}: gram rel {e:.3e}")
    assert e <= 4 * _kappa(want) * EPS_BF16
    assert e <= 3e-5
    if xdt == torch.bfloat16:
        Rp, _ = hip.fold_finalize(None, 0, X, 1 / math.sqrt(p), lam, torch.float32, 1)
        assert e <= _gram_rel(Rp, want)


def test_fold_finalize_gram_flags(hip):
    """Rank deficiency without damping and non-finite input give status 2; the panel
    path then gives its own flag; a well-posed call after them is unaffected."""
    g = torch.Generator(device=DEV).manual_seed(5)
    X = torch.randn(900, 600, device=DEV, generator=g)
    X[:, 37] = 0.0
    _, st = hip.fold_finalize(None, 0, X, 1 / 30.0, 0.0, torch.float32, 1, gram=True)
    assert st.item() == 2
    X2 = torch.randn(3000, 2200, device=DEV, generator=g)
    X2[:, 1900] = 3.0 * X2[:, 12] - X2[:, 1400]   # dependent columns in different blocks
    _, st = hip.fold_finalize(None, 0, X2, 1 / math.sqrt(3000), 0.0, torch.float32, 1, gram=True)
    assert st.item() == 2
    # one row under damping 1e-2: A = x x^T + 1e-2 I; the pivot of a column with
    # x_j^2 = 16 is about 1e-2 (1 + ...) of its diagonal 16.01, i.e. < 1e-3 of it
    x = torch.ones(1, 600, device=DEV)
    x[0, 300] = 4.0
    _, st = hip.fold_finalize(None, 0, x, 1.0, 1e-2, torch.float32, 1, gram=True)
    assert st.item() == 2
    x[0, 300] = 1.0   # every pivot ratio about 1e-2 / 1.01: above the threshold
    Rx, st = hip.fold_finalize(None, 0, x, 1.0, 1e-2, torch.float32, 1, gram=True)
    assert st.item() == 1
    assert _gram_rel(Rx, O.chol_factor([_bf16_np(x)], 1, 1e-2)) <= 3e-5
    X3 = torch.randn(900, 600, device=DEV, generator=g)
    X3[5, 5] = float("nan")
    _, st = hip.fold_finalize(None, 0, X3, 1 / 30.0, 1e-2, torch.float32, 1, gram=True)
    assert st.item() == 2
    _, fl = hip.fold_finalize(None, 0, X3, 1 / 30.0, 1e-2, torch.float32, 1)
    assert fl.item() == 0
    X3[5, 5] = 0.5
    Rd, st = hip.fold_finalize(None, 0, X3, 1 / 30.0, 1e-2, torch.float32, 1, gram=True)
    want = O.chol_factor([_bf16_np(X3)], 900, 1e-2)
    assert st.item() == 1 and _gram_rel(Rd, want) <= 3e-5


def test_fold_finalize_gram_guards(hip):
    X = torch.randn(10, 20, device=DEV)
    with pytest.raises(Exception):   # fewer rows than columns and no damping
        hip.fold_finalize(None, 0, X, 1.0, 0.0, torch.float32, 1, gram=True)
    with pytest.raises(Exception):   # bf16 arithmetic only
        hip.fold_finalize(None, 0, X, 1.0, 1e-2, torch.float32, 0, gram=True)


def test_fold_finalize_gram_is_deterministic(hip):
    g = torch.Generator(device=DEV).manual_seed(11)
    X = torch.randn(3000, 3300, device=DEV, generator=g).to(torch.bfloat16)
    a, _ = hip.fold_finalize(None, 0, X, 1 / math.sqrt(3000), 1e-2, torch.bfloat16, 1, gram=True)
    b, _ = hip.fold_finalize(None, 0, X, 1 / math.sqrt(3000), 1e-2, torch.bfloat16, 1, gram=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("B,prev,p,n", [(3, 0, 900, 600), (4, 0, 4096, 3100), (2, 1200, 1200, 2100),
                                        (4, 0, 8192, 4096)])
def test_fold_finalize_gram_batched_matches_single(hip, B, prev, p, n):
    """The batched entry (one chain of launches for B same-shape sides) gives every
    entry exactly the bits of the single-side entry, status and kappa bound included."""
    g = torch.Generator(device=DEV).manual_seed(B * 7 + n)
    Xs = [(torch.randn(p, n, device=DEV, generator=g) * (1 + e)).to(torch.bfloat16)
          for e in range(B)]
    Rs = None
    r = 0
    if prev:
        Rs = []
        for e in range(B):
            R, r = _fold_chunks(hip, [torch.randn(prev, n, device=DEV, generator=g)], n)
            Rs.append(R)
    rows = prev + p
    out, st, kb = hip.fold_finalize_gram_batched(Rs, r, Xs, 1 / math.sqrt(rows), 1e-2,
                                                 torch.bfloat16)
    for e in range(B):
        one, s1, k1 = hip.fold_finalize(Rs[e] if Rs else None, r, Xs[e], 1 / math.sqrt(rows), 1e-2,
                                        torch.bfloat16, 1, gram=True, with_kappa=True)
        assert torch.equal(out[e], one), e
        assert st[e].item() == s1.item() == 1
        assert kb[e].item() == k1.item()
