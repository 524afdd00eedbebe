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


# ---------------------------------------------------------------------------
# the streaming fold by the Gram route (ifk_tsqr_fold_gram)
# ---------------------------------------------------------------------------
FOLD_TOL = 1e-4


@pytest.mark.parametrize("prev,p,n,xdt", [
    ([], 600, 500, torch.float32), ([300], 400, 600, torch.bfloat16), ([600], 600, 600, torch.float32),
    ([1200], 1200, 2100, torch.float32), ([512, 512], 512, 1024, torch.bfloat16),
    ([2048], 4096, 3072, torch.float32),
])
def test_tsqr_fold_gram_matches_closed_form(hip, prev, p, n, xdt):
    """R <- the undamped factor of [R_in; bf16(X)] (the running factor enters as
    fp32 state, split hi + lo; the chunk as the bf16 operand it is):
    ||R^T R - P^T P||_F / ||P^T P||_F <= 3e-5 (Cholesky's backward error with
    2^-17 products), upper triangular with a positive diagonal, and no worse than
    the bf16 panel fold of the same chunk against the same closed form."""
    g = torch.Generator(device=DEV).manual_seed(p + n + len(prev))
    R, r = _fold_chunks(hip, [torch.randn(q, n, device=DEV, generator=g) for q in prev], n)
    X = torch.randn(p, n, device=DEV, generator=g).to(xdt)
    R_before = R.clone()
    st = hip.fold_gram_(R, r, X, FOLD_TOL)
    assert st.item() == 1
    parts = ([R_before[:r].double().cpu().numpy()] if r > 0 else []) + [_bf16_np(X)]
    want = O.chol_factor(parts, 1, 0.0)
    e = _gram_rel(R, want)
    Rp = R_before.clone()
    assert hip.fold_(Rp, r, X, 1) == n
    ep = _gram_rel(Rp, want)
    print(f"tsqr_fold_gram n={n} p={p} r_in={r}: gram rel {e:.3e} (panel fold {ep:.3e})")
    assert e <= 3e-5 and e <= ep
    Rg = R.double().cpu().numpy()
    assert np.all(np.diag(Rg) > 0) and not np.any(np.tril(Rg, -1))


def test_tsqr_fold_gram_refusals_leave_R(hip):
    """A dependent column (pivot ratio 0), a NaN, and a nearly square running
    factor whose last pivot ratio is below the threshold: status 2 and R bit for bit
    as it was; the panel fold then takes the chunk."""
    from ifkfac_amd.activation_hooks import fold_chunk
    g = torch.Generator(device=DEV).manual_seed(21)
    R, r = _fold_chunks(hip, [torch.randn(700, 640, device=DEV, generator=g)], 640)
    X = torch.randn(300, 640, device=DEV, generator=g)
    for case in ("dependent", "nan"):
        Rz = torch.zeros(640, 640, device=DEV)
        Y = X.clone()
        if case == "dependent":
            Y = torch.randn(900, 640, device=DEV, generator=g)
            Y[:, 600] = 2.0 * Y[:, 3] - Y[:, 500]
            before = Rz.clone()
            assert hip.fold_gram_(Rz, 0, Y, FOLD_TOL).item() == 2
            assert torch.equal(Rz, before)
        else:
            Y[17, 33] = float("nan")
            before = R.clone()
            assert hip.fold_gram_(R, r, Y, FOLD_TOL).item() == 2
            assert torch.equal(R, before)
    # kappa 1e2 chunks of 512 rows into a 1024-column factor: the second fold is
    # square with a pivot ratio near 3e-6 (refused), the later ones near 3e-3
    rng = np.random.default_rng(1)
    Xk = torch.from_numpy(O.kappa_matrix(4096, 1024, 1e2, rng).astype(np.float32))
    Xk = Xk.to(torch.bfloat16).to(DEV)
    Rg = torch.zeros(1024, 1024, device=DEV)
    Rp = torch.zeros(1024, 1024, device=DEV)
    rg = rp = 0
    statuses = []
    for c in range(8):
        chunk = Xk[512 * c:512 * (c + 1)]
        if rg + 512 >= 1024:
            Rb = Rg.clone()
            s = hip.fold_gram_(Rb, rg, chunk, FOLD_TOL).item()
            statuses.append(s)
        rg = fold_chunk(Rg, rg, chunk, 1)
        rp = hip.fold_(Rp, rp, chunk, 1)
    print(f"kappa 1e2 chunk statuses {statuses}")
    assert statuses[0] == 2 and all(s == 1 for s in statuses[1:])
    want = O.chol_factor([_bf16_np(Xk)], 1, 0.0)
    eg, ep = _gram_rel(Rg, want), _gram_rel(Rp, want)
    print(f"8 folds: gram route {eg:.3e}, panel folds {ep:.3e}")
    assert rg == rp == 1024 and eg <= ep


def test_tsqr_fold_gram_guards(hip):
    R = torch.zeros(64, 64, device=DEV)
    with pytest.raises(Exception):   # the folded factor would not be square
        hip.fold_gram_(R, 10, torch.randn(50, 64, device=DEV), FOLD_TOL)
    with pytest.raises(Exception):   # tolerance outside (0, 1)
        hip.fold_gram_(R, 0, torch.randn(80, 64, device=DEV), 0.0)


# ---------------------------------------------------------------------------
# the inverse formed beside the factorisation (ifk_fold_finalize_gram_inverse)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("B,prev,p,n,odt", [
    (1, 0, 500, 300, torch.bfloat16), (1, 0, 2000, 1500, torch.float32),
    (1, 1200, 1200, 2100, torch.bfloat16), (1, 0, 4000, 3100, torch.bfloat16),
    (1, 0, 6000, 5000, torch.float32), (3, 0, 2600, 2100, torch.bfloat16),
    (2, 0, 4096, 4096, torch.bfloat16),
])
def test_fold_finalize_gram_inverse(hip, B, prev, p, n, odt):
    """Factor, status and kappa bound bit for bit those of the call without the
    inverse; Zb = bf16(Z) and ZT = bf16(Z^T) exactly with the other triangle zero;
    ||R Z - I||_max, R the fp32 factor, at most twice that of ifk_tri_inverse_bf16
    on the same R (both bf16 arithmetic) plus 1e-3."""
    g = torch.Generator(device=DEV).manual_seed(B * 13 + n)
    Xs = [(torch.randn(p, n, device=DEV, generator=g) * (1 + e)).to(torch.bfloat16)
          for e in range(B)]
    Rs, r = None, 0
    if prev:
        Rs = []
        for e in range(B):
            R, r = _fold_chunks(hip, [torch.randn(prev, n, device=DEV, generator=g)], n)
            Rs.append(R)
    rows = prev + p
    out, st, kb, (Z, Zb, ZT) = hip.fold_finalize_gram_batched(Rs, r, Xs, 1 / math.sqrt(rows),
                                                             1e-2, odt, with_inverse=True)
    out0, st0, kb0 = hip.fold_finalize_gram_batched(Rs, r, Xs, 1 / math.sqrt(rows), 1e-2, odt)
    assert torch.equal(out, out0) and torch.equal(st, st0) and torch.equal(kb, kb0)
    R32, _, _ = hip.fold_finalize_gram_batched(Rs, r, Xs, 1 / math.sqrt(rows), 1e-2,
                                               torch.float32)
    eye = torch.eye(n, device=DEV, dtype=torch.float64)
    for e in range(B):
        assert st[e].item() == 1
        assert torch.equal(Zb[e], Z[e].to(torch.bfloat16))
        assert torch.equal(ZT[e], Z[e].t().contiguous().to(torch.bfloat16))
        assert torch.count_nonzero(torch.tril(Z[e], -1)).item() == 0
        Rd = R32[e].double()
        err = (Rd @ Z[e].double() - eye).abs().max().item()
        Zt, _, _ = hip.tri_inverse_bf16(R32[e])
        err_t = (Rd @ Zt.double() - eye).abs().max().item()
        print(f"B={B} n={n} entry {e}: ||R Z - I||_max {err:.3e} (tri_inverse_bf16 {err_t:.3e})")
        assert err <= 2 * err_t + 1e-3


def test_release_stream_state(hip):
    """ifk_release_stream_state: a stream's helper set (three streams and their
    events) released between two factorisations of more than 1024 columns gives
    the second the same bits;
    releasing a stream with no set, or twice, is a no-op."""
    g = torch.Generator(device=DEV).manual_seed(41)
    X = torch.randn(4000, 3100, device=DEV, generator=g).to(torch.bfloat16)
    st_ = torch.cuda.Stream()
    with torch.cuda.stream(st_):
        a, s1 = hip.fold_finalize(None, 0, X, 1 / math.sqrt(4000), 1e-2, torch.bfloat16, 1,
                                  gram=True)
        hip.release_stream_state(DEV, st_)
        hip.release_stream_state(DEV, st_)
        b, s2 = hip.fold_finalize(None, 0, X, 1 / math.sqrt(4000), 1e-2, torch.bfloat16, 1,
                                  gram=True)
        hip.release_stream_state(DEV, st_)
    torch.cuda.synchronize()
    assert s1.item() == s2.item() == 1 and torch.equal(a, b)
    hip.release_stream_state(DEV, torch.cuda.Stream())


def test_gram_route_products_own_kernel(hip):
    """The Gram route's large products (Gram columns, band and panel updates: N =
    1024 column blocks) run on this library's direct-to-LDS kernel (variant bit
    6), data-parallel or stream-K (bit 9) as the dispatcher estimates faster
    (at n = 3100, p = 4000 every one is short enough for data-parallel), and
    the factor meets the fp64 closed form at 3e-5."""
    import ctypes
    from ifkfac_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=DEV).manual_seed(29)
    p, n = 4000, 3100
    X = torch.randn(p, n, device=DEV, generator=g).to(torch.bfloat16)
    Xd = _bf16_np(X)
    Ro = np.linalg.cholesky(Xd.T @ Xd / p + 1e-2 * np.eye(n)).T
    torch.cuda.synchronize()
    _lib.check(lib.ifk_profile_begin(-2), "profile_begin")
    R, st = hip.fold_finalize(None, 0, X, 1 / math.sqrt(p), 1e-2, torch.float32, 1, gram=True)
    torch.cuda.synchronize()
    cnt = ctypes.c_int64(0)
    _lib.check(lib.ifk_profile_end(ctypes.byref(cnt)), "profile_end")
    v, ms, fl, by = ctypes.c_int(), ctypes.c_float(), ctypes.c_double(), ctypes.c_double()
    m_, n_, k_ = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    variants = []
    for i in range(cnt.value):
        _lib.check(lib.ifk_profile_get(i, *(ctypes.byref(x) for x in (v, ms, fl, by, m_, n_, k_))),
                   "profile_get")
        variants.append((v.value, m_.value, n_.value, k_.value))
    assert int(st.reshape(-1)[0].item()) == 1
    sk = [x for x in variants if (x[0] >> 9) & 1]
    print(f"{len(variants)} GEMM launches, {len(sk)} stream-K; closed form "
          f"{_gram_rel(R.double().cpu().numpy(), Ro):.2e}")
    assert len(variants) >= 10
    # the dispatcher's rule: products of 1e9 multiply-adds or more on the
    # direct-to-LDS kernel (the ragged last block's smaller ones on the
    # 128 x 128 engine)
    big = [x for x in variants if x[1] * x[2] * x[3] >= 1e9]
    assert len(big) >= 8 and all((x[0] >> 6) & 1 for x in big)
    assert _gram_rel(R.double().cpu().numpy(), Ro) <= 3e-5


def test_gram_route_repeated_folds_identical(hip):
    """Ten folds of the same chunk into the same square factor, each a Gram-route
    factorisation on three streams (n = 3072: the helper and Gram streams run
    stream-K products beside the chain), give identical bits: each stream has
    its own counters and partial tiles, and a stream-K tile's sum does not
    depend on the order its shares arrive in."""
    g = torch.Generator(device=DEV).manual_seed(31)
    n, p = 3072, 4096
    R0 = torch.zeros(n, n, device=DEV)
    assert hip.fold_gram_(R0, 0, torch.randn(p, n, device=DEV, generator=g), 1e-4).item() == 1
    X = torch.randn(p, n, device=DEV, generator=g)
    outs = []
    for _ in range(10):
        R = R0.clone()
        st = hip.fold_gram_(R, n, X, 1e-4)
        outs.append((st.item(), R))
    assert all(s == 1 for s, _ in outs)
    for _, R in outs[1:]:
        assert torch.equal(R, outs[0][1])
