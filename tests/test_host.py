"""Host logic of ifkfac_amd on the CPU, with the oracle-backed test double.

The real IFKFAC / RawActivationHooks code runs; only the numerical seams are
answered by the oracle (tests/oracle_backend.py).  These tests pin the
reference's control flow: the factor schedule (ifkfac.py:560-564), skip and
clear rules (activation_hooks.py:262-311, ifkfac.py:209-237), layer
classification and per-layer update (ifkfac.py:330-423, :443-519), capture
controls, batched / deferred modes and the EMA blend (ifkfac.py:261-285).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import ifk_oracle as O
from oracle_backend import OracleBackend


@pytest.fixture
def be():
    from ifkfac_amd import _backend
    b = OracleBackend()
    prev = _backend.set_backend(b)
    yield b
    _backend.set_backend(prev)


def _mlp(seed=0, bias=True):
    torch.manual_seed(seed)
    return nn.Sequential(nn.Linear(8, 16, bias=bias), nn.ReLU(), nn.Linear(16, 4, bias=bias))


def _capture(model, X):
    """Inputs and output-gradients of every Linear, recorded independently."""
    acts, grads = {}, {}
    hs = []
    for m in model.modules():
        if isinstance(m, nn.Linear):
            hs.append(m.register_forward_hook(lambda mod, i, o: acts.__setitem__(mod, i[0].detach().clone())))
            hs.append(m.register_full_backward_hook(lambda mod, gi, go: grads.__setitem__(mod, go[0].detach().clone())))
    return acts, grads, hs


def test_single_step_matches_oracle(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    X = torch.randn(64, 8, generator=torch.Generator().manual_seed(1))
    Y = torch.randint(0, 4, (64,), generator=torch.Generator().manual_seed(2))
    lr, lam = 1e-2, 1e-2
    opt = IFKFAC(model, lr=lr, damping=lam, factor_update_freq=1, momentum=0.9)
    acts, grads, hs = _capture(model, X)
    W0 = {m: (m.weight.detach().clone(), m.bias.detach().clone()) for m in opt.hooks.linear_layers}
    loss = F.cross_entropy(model(X), Y)
    opt.zero_grad()
    loss.backward()
    gW = {m: (m.weight.grad.clone(), m.bias.grad.clone()) for m in opt.hooks.linear_layers}
    opt.step()
    for h in hs:
        h.remove()
    for m in opt.hooks.linear_layers:
        x = acts[m].double().numpy()
        d = grads[m].double().numpy()
        R_X = O.get_factor(O.streaming_tsqr_update(None, x), x.shape[0], lam)
        R_G = O.get_factor(O.streaming_tsqr_update(None, d), d.shape[0], lam)
        nat = O.apply_vered(gW[m][0].double().numpy(), R_X, R_G)
        nat_b = O.apply_vered_bias(gW[m][1].double().numpy(), R_G)
        want_W = W0[m][0].double().numpy() - lr * nat      # momentum buffer starts at nat
        want_b = W0[m][1].double().numpy() - lr * nat_b    # bias: no momentum
        assert np.abs(m.weight.detach().double().numpy() - want_W).max() < 1e-5
        assert np.abs(m.bias.detach().double().numpy() - want_b).max() < 1e-5


def test_schedule_every_freq_steps(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=10)
    X = torch.randn(64, 8)
    for step in range(1, 26):
        opt.zero_grad()
        model(X).pow(2).mean().backward()
        before = be.calls["finalize"] + be.calls["fold_finalize"]
        opt.step()
        fired = be.calls["finalize"] + be.calls["fold_finalize"] > before
        assert fired == O.should_update_factors(step, 10), step


def test_narrow_batch_layer_is_skipped_and_gets_plain_sgd(be):
    """p < n: layer skipped, plain SGD without momentum and without bias update."""
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(64, 8), nn.ReLU(), nn.Linear(8, 4))
    opt = IFKFAC(model, lr=0.1, factor_update_freq=1, momentum=0.9)
    X = torch.randn(16, 64)          # 16 rows < n_in = 64 for the first layer
    first, second = model[0], model[2]
    for _ in range(3):
        W = first.weight.detach().clone()
        b = first.bias.detach().clone()
        opt.zero_grad()
        model(X).pow(2).mean().backward()
        g = first.weight.grad.clone()
        opt.step()
        assert first not in opt._factors and second in opt._factors
        assert torch.allclose(first.weight, W - 0.1 * g, atol=1e-7)
        assert torch.equal(first.bias, b)                 # not updated
        assert first not in opt._momentum_buffers
        # hooks.clear() after the successful update wiped the partial factor
        assert opt.hooks._R_X[first] is None


def test_non_finite_factor_is_dropped(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=1)
    X = torch.randn(64, 8)
    X[3, 2] = float("nan")
    opt.zero_grad()
    model(X).pow(2).mean().backward()
    opt.step()
    assert model[0] not in opt._factors


def test_momentum_and_weight_decay_two_steps(be):
    from ifkfac_amd import IFKFAC
    model = _mlp(bias=False)
    lr, mu, wd, lam = 5e-2, 0.9, 0.1, 1e-2
    opt = IFKFAC(model, lr=lr, damping=lam, factor_update_freq=1, momentum=mu, weight_decay=wd)
    X = torch.randn(64, 8, generator=torch.Generator().manual_seed(3))
    layer = model[2]
    buf = None
    W = layer.weight.detach().double().numpy().copy()
    for _ in range(2):
        acts, grads, hs = _capture(model, X)
        opt.zero_grad()
        model(X).pow(2).mean().backward()
        g = layer.weight.grad.double().numpy()
        opt.step()
        for h in hs:
            h.remove()
        x, d = acts[layer].double().numpy(), grads[layer].double().numpy()
        R_X = O.get_factor(O.streaming_tsqr_update(None, x), 64, lam)
        R_G = O.get_factor(O.streaming_tsqr_update(None, d), 64, lam)
        nat = O.apply_vered(g, R_X, R_G)
        buf = nat if buf is None else mu * buf + nat
        W = W * (1 - lr * wd) - lr * buf
        assert np.abs(layer.weight.detach().double().numpy() - W).max() < 1e-5


def test_grad_clip_scales_natural_gradient(be):
    from ifkfac_amd import IFKFAC
    model = _mlp(bias=False)
    opt = IFKFAC(model, lr=1.0, factor_update_freq=1, momentum=0.0, grad_clip=1e-3)
    X = torch.randn(64, 8)
    W = [m.weight.detach().clone() for m in opt.hooks.linear_layers]
    opt.zero_grad()
    model(X).pow(2).mean().backward()
    opt.step()
    for m, w in zip(opt.hooks.linear_layers, W):
        step = (m.weight.detach() - w).norm().item()
        assert step == pytest.approx(1e-3, rel=1e-4)


def test_grad_clip_only_clips_the_weight_natural_gradient(be):
    """grad_clip scales a weight's natural gradient only (ifkfac/ifkfac.py:397-400,
    494-497); bias updates (:418-423, :515-519) and the plain-SGD step of a layer
    without factors (:443-448) are never clipped.  With factor_update_freq=2,
    step 1 has no factors (plain SGD on the weight, bias untouched) and step 2
    builds them from both steps' rows: its weight step has norm lr * grad_clip and
    its bias step is the oracle's unclipped G^-1 g_b."""
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    layer = nn.Linear(8, 4, bias=True)
    model = nn.Sequential(layer)
    lr, lam, clip = 0.5, 1e-2, 1e-3
    opt = IFKFAC(model, lr=lr, damping=lam, factor_update_freq=2, momentum=0.0, grad_clip=clip)
    g = torch.Generator().manual_seed(1)
    deltas = []
    for step, X in enumerate([torch.randn(64, 8, generator=g), torch.randn(64, 8, generator=g)]):
        acts, grads, hs = _capture(model, X)
        W, b = layer.weight.detach().clone(), layer.bias.detach().clone()
        opt.zero_grad()
        model(X).pow(2).mean().backward()
        gW, gb = layer.weight.grad.clone(), layer.bias.grad.clone()
        for h in hs:
            h.remove()
        deltas.append(grads[layer].double().numpy())
        opt.step()
        if step == 0:   # no factors: plain SGD, unclipped, bias untouched
            assert torch.allclose(layer.weight.detach(), W - lr * gW, atol=1e-7)
            assert (lr * gW).norm().item() > 10 * clip
            assert torch.equal(layer.bias.detach(), b)
    step_w = (layer.weight.detach() - W).norm().item()
    assert step_w == pytest.approx(lr * clip, rel=1e-4)       # the weight step is clipped
    d = np.vstack(deltas)
    R_G = O.get_factor(O.streaming_tsqr_update(None, d), d.shape[0], lam)
    want_b = b.double().numpy() - lr * O.apply_vered_bias(gb.double().numpy(), R_G)
    assert np.abs(layer.bias.detach().double().numpy() - want_b).max() < 1e-6
    assert (layer.bias.detach() - b).norm().item() > 10 * clip  # and the bias step is not


def test_weight_step_rounds_once_for_bf16_parameters(be):
    """A non-fp32 weight takes W.add_(nat, alpha=-lr) with the fp32 natural
    gradient: one rounding to bf16, as torch does for the reference's update
    (ifkfac/ifkfac.py:413), not a cast of nat to bf16 first."""
    from ifkfac_amd import IFKFAC
    layer = nn.Linear(8, 4, bias=False)
    opt = IFKFAC(nn.Sequential(layer), lr=0.3, factor_update_freq=1, momentum=0.0)
    layer.weight.data = torch.zeros(4, 8, dtype=torch.bfloat16)
    nat = torch.full((4, 8), 1.0 + 3 * 2 ** -9)        # not a bf16 value
    opt._update_param(layer.weight, nat, 0.3, 0.0, 0.0, None)
    want = torch.zeros(4, 8, dtype=torch.bfloat16).add_(nat, alpha=-0.3)
    twice = torch.zeros(4, 8, dtype=torch.bfloat16).add_(nat.bfloat16(), alpha=-0.3)
    assert torch.equal(layer.weight.detach(), want)
    assert not torch.equal(want, twice)                  # the check tells the two apart


def test_bf16_mode_chooses_solve_arithmetic_by_kappa(be):
    """use_true_bf16: a layer whose factors are near-isotropic (kappa_2 <= 1.5,
    the damping dominating its Grams) keeps the bf16 inverse copies and apply; a
    layer whose input carries a large mean (kappa(R_X) far above 1.5) gets fp32
    inverses applied through their split bf16 halves, fp32 accuracy to about
    2^-17 per product, the reference's bf16-mode arithmetic being fp32 solves
    (triangular.py:621-628).  The update matches the oracle's closed form to
    2 * 2^-17 kappa(R_X) kappa(R_G) (measured 3e-4 at kappa(R_X) = 140, inside
    the bf16-mode natural-gradient bound 2e-2); an apply that dropped the lo
    halves would miss it by two orders of magnitude."""
    from ifkfac_amd import IFKFAC
    from ifkfac_amd._backend import MATH_BF16, MATH_F32
    torch.manual_seed(0)
    iso, skew = nn.Linear(8, 4, bias=False), nn.Linear(8, 4, bias=False)
    lam = 1.0
    opt_iso = IFKFAC(nn.Sequential(iso), lr=1.0, damping=lam, factor_update_freq=1, momentum=0.0,
                     use_true_bf16=True)
    g = torch.Generator().manual_seed(3)
    X = torch.randn(64, 8, generator=g) * 0.1
    iso(X).pow(2).mean().backward()
    opt_iso.step()
    assert opt_iso._solve_math[iso] == MATH_BF16 and iso in opt_iso._inverse_copies
    assert max(opt_iso._kappas[iso]) <= 1.5
    opt_sk = IFKFAC(nn.Sequential(skew), lr=1.0, damping=1e-2, factor_update_freq=1,
                    momentum=0.0, use_true_bf16=True)
    Xs = torch.randn(64, 8, generator=g) + 5.0
    acts, grads, hs = _capture(nn.Sequential(skew), Xs)
    W0 = skew.weight.detach().clone()
    skew(Xs).pow(2).mean().backward()
    gW = skew.weight.grad.double().numpy()
    for h in hs:
        h.remove()
    opt_sk.step()
    assert opt_sk._solve_math[skew] == MATH_F32 and skew not in opt_sk._inverse_copies
    assert opt_sk._kappas[skew][0] > 1.5
    RX, RG = (f.float().double().numpy() for f in opt_sk._factors[skew])
    want = W0.double().numpy() - O.apply_vered(gW, RX, RG)
    assert skew in opt_sk._split_copies
    err = np.abs(skew.weight.detach().double().numpy() - want).max() / np.abs(want).max()
    kx, kg = opt_sk._kappas[skew]
    assert err < 2 * 2.0 ** -17 * kx * kg


def test_capture_controls(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=100)
    X = torch.randn(64, 8)
    opt.pause_capture()
    model(X).sum().backward()
    assert be.calls["fold"] == 0
    with opt.capture():
        model(X).sum().backward()
    assert be.calls["fold"] == 4           # 2 layers x (X, G)
    model(X).sum().backward()
    assert be.calls["fold"] == 4           # paused again after the block
    opt.resume_capture()
    model(X).sum().backward()
    assert be.calls["fold"] == 8


def test_max_out_dim_layers_untracked_and_never_updated(be):
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(8, 16), nn.ReLU(), nn.Linear(16, 40))
    opt = IFKFAC(model, lr=1e-2, factor_update_freq=1, max_out_dim=32)
    assert opt.hooks.linear_layers == [model[0]]
    W = model[2].weight.detach().clone()
    model(torch.randn(64, 8)).pow(2).mean().backward()
    opt.step()
    assert torch.equal(model[2].weight, W)


def _factors_for_mode(be, **kw):
    from ifkfac_amd import RawActivationHooks
    model = _mlp(seed=4)
    hooks = RawActivationHooks(model, damping=1e-2, **kw)
    hooks.enable()
    g = torch.Generator().manual_seed(5)
    for _ in range(3):
        model(torch.randn(16, 8, generator=g)).pow(2).mean().backward()
    hooks.flush()
    return {i: f for i, f in enumerate(hooks.get_factors().values())}


def test_modes_agree(be):
    a = _factors_for_mode(be)
    b = _factors_for_mode(be, batched=True)
    c = _factors_for_mode(be, deferred=True, deferred_window=2)
    assert a.keys() == b.keys() == c.keys() and len(a) == 2
    for i in a:
        for k in range(2):
            assert torch.allclose(a[i][k], b[i][k], atol=1e-5)
            assert torch.allclose(a[i][k], c[i][k], atol=1e-5)


def test_batched_and_deferred_are_exclusive(be):
    from ifkfac_amd import RawActivationHooks
    with pytest.raises(ValueError):
        RawActivationHooks(_mlp(), batched=True, deferred=True)


def test_batched_rank_error_keeps_state(be):
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(32, 8))
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=1, batched_qr=True)
    model(torch.randn(8, 32)).pow(2).mean().backward()
    opt.step()                                 # 8 rows < 32: IFKFACRankError -> skipped
    assert opt._factors == {}
    assert opt.hooks._n_rows_X[model[0]] == 8  # state kept for the next window


def test_gamma_blend_is_exact(be):
    from ifkfac_amd import IFKFAC
    model = _mlp(bias=False)
    opt = IFKFAC(model, lr=0.0, factor_update_freq=1, gamma=0.5)
    X1, X2 = torch.randn(64, 8), torch.randn(64, 8)
    model(X1).pow(2).mean().backward()
    opt.step()
    old = {m: f[0].double() for m, f in opt._factors.items()}
    opt.zero_grad()
    model(X2).pow(2).mean().backward()
    fresh = {i: f[0].double() for i, f in enumerate(opt.hooks.get_factors().values())}
    opt.step()
    for i, (m, f) in enumerate(opt._factors.items()):
        R_b = f[0].double()
        want = 0.5 * old[m].T @ old[m] + 0.5 * fresh[i].T @ fresh[i]
        assert torch.allclose(R_b.T @ R_b, want, atol=1e-5)


def test_true_bf16_stores_rne_bf16_factors(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=1, use_true_bf16=True)
    X = torch.randn(64, 8)
    model(X).pow(2).mean().backward()
    fp32 = {i: f for i, f in enumerate(opt.hooks.get_factors().values())}
    opt.step()
    for i, (m, (R_X, R_G)) in enumerate(opt._factors.items()):
        assert R_X.dtype == torch.bfloat16 and R_G.dtype == torch.bfloat16
        assert torch.equal(R_X, fp32[i][0].to(torch.bfloat16))


def test_conv2d_layer_uses_im2col_rows(be):
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    model = nn.Sequential(nn.Conv2d(3, 4, 3), nn.ReLU(), nn.Flatten(), nn.Linear(4 * 6 * 6, 5))
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=1, max_conv_rows=0)
    model(torch.randn(8, 3, 8, 8)).pow(2).mean().backward()
    assert opt.hooks._n_rows_X[model[0]] == 8 * 36
    assert opt.hooks._running_factor(model[0], "X").shape == (27, 27)
    W = model[0].weight.detach().clone()
    opt.step()
    assert model[0] in opt._factors
    assert model[0].weight.shape == W.shape and not torch.equal(model[0].weight, W)


def test_augment_bias_factor_has_extra_column(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=1, augment_bias=True)
    model(torch.randn(64, 8)).pow(2).mean().backward()
    opt.step()
    R_X, _ = opt._factors[model[0]]
    assert R_X.shape == (9, 9)


def test_sequence_inputs_are_subsampled(be):
    from ifkfac_amd import RawActivationHooks
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(8, 8))
    hooks = RawActivationHooks(model, max_seq_rows=50)
    hooks.enable()
    model(torch.randn(4, 30, 8)).pow(2).mean().backward()
    assert hooks._n_rows_X[model[0]] == 50 and hooks._n_rows_G[model[0]] == 50


def test_timing_and_repr(be):
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=1)
    model(torch.randn(64, 8)).pow(2).mean().backward()
    opt.step()
    stats = opt.get_timing_stats()
    assert set(stats) == {"factor_compute", "precondition", "total_step"}
    assert stats["total_step"]["count"] == 1
    assert repr(opt).startswith("IFKFAC(damping=0.01, factor_update_freq=1")
    opt.cleanup()
    assert opt._factors == {} and not opt.hooks.is_enabled


# --------------------------------------------------------------------------- reference trajectories


def _golden():
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_trajectories.npz"))


@pytest.mark.parametrize("mode", ["fp32", "bf16"])
def test_demo_trajectory_matches_reference_run(be, mode):
    """Host logic + oracle numerics reproduce the reference's own 100-step run
    (tests/golden/make_reference_trajectories.py).  The first ten losses agree to
    1e-5 in fp32 mode; in bf16 mode to 5e-5, the layers whose kappa bound exceeds
    1.5 being applied through split bf16 inverses (2^-17 per product where the
    reference solves in fp32; measured 1.2e-5)."""
    import sys, os, contextlib, io
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_reference_trajectories as M
    from ifkfac_amd import IFKFAC
    ref = _golden()
    with contextlib.redirect_stdout(io.StringIO()):
        losses, final, *_ = M.demo(IFKFAC, mode == "bf16")
    want = ref[f"demo_{mode}_losses"]
    assert np.all(np.abs(losses - want) <= 2e-3 * np.abs(want) + 1e-7)
    tol10 = 1e-5 if mode == "fp32" else 5e-5
    assert np.all(np.abs(losses[:10] - want[:10]) <= tol10 * np.abs(want[:10]))
    if mode == "fp32":
        for i, w in enumerate(final):
            rw = ref[f"demo_fp32_final_{i}"]
            assert np.linalg.norm(w - rw) / np.linalg.norm(rw) < 1e-5


@pytest.mark.parametrize("name", ["canary", "canary_bias"])
def test_canary_runs_match_reference_including_divergence(be, name):
    """The reference's own canary configurations diverge on this torch version;
    the same host logic reproduces the trajectory up to and including that."""
    import sys, os, contextlib, io
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    import make_reference_trajectories as M
    from ifkfac_amd import IFKFAC
    want = _golden()[f"{name}_losses"]
    with contextlib.redirect_stdout(io.StringIO()), np.errstate(all="ignore"):
        got = getattr(M, name)(IFKFAC)
    ok = np.isfinite(want) & (np.abs(want) < 1e3)
    assert ok.sum() >= 10
    assert np.all(np.abs(got[ok] - want[ok]) <= 1e-4 * np.abs(want[ok]))
    assert not np.isfinite(got[-1]) and not np.isfinite(want[-1])


def test_update_step_consumes_held_chunk_in_fused_call(be):
    """Before an update step the hooks hold the last chunk back, and the factor
    update folds and finalizes it in one fused call; the factors equal the
    closed form of every chunk of the window (two backward passes here)."""
    from ifkfac_amd import IFKFAC
    model = _mlp()
    lam = 1e-2
    opt = IFKFAC(model, lr=1e-3, damping=lam, factor_update_freq=1)
    gen = torch.Generator().manual_seed(5)
    Xs = [torch.randn(40, 8, generator=gen), torch.randn(30, 8, generator=gen)]
    acts, grads, hs = _capture(model, Xs[0])
    seen = {m: ([], []) for m in opt.hooks.linear_layers}
    opt.zero_grad()
    for X in Xs:
        model(X).pow(2).mean().backward()
        for m in opt.hooks.linear_layers:
            seen[m][0].append(acts[m].double().numpy())
            seen[m][1].append(grads[m].double().numpy())
    for h in hs:
        h.remove()
    first = opt.hooks.linear_layers[0]
    assert opt.hooks._held_X[first] is not None           # the second chunk is held
    assert be.calls["fold"] == 4                           # the first chunk of each side folded
    opt.step()
    assert be.calls["fold_finalize"] == 4 and be.calls["finalize"] == 0
    for m in opt.hooks.linear_layers:
        R_X, R_G = opt._factors[m]
        want_X = O.chol_factor(seen[m][0], 70, lam)
        want_G = O.chol_factor(seen[m][1], 70, lam)
        assert np.abs(R_X.double().numpy() - want_X).max() < 1e-5
        assert np.abs(R_G.double().numpy() - want_G).max() < 1e-5
    assert opt.hooks._held_X[first] is None and opt.hooks._R_X[first] is None


def test_update_step_recomputes_ill_conditioned_cqr_side(be):
    """The fused factor update runs the CholeskyQR2 variant; a side that reports
    an ill-conditioned block (status 2) is recomputed by the panel path before
    the factors are used, so they still equal the closed form."""
    from ifkfac_amd import IFKFAC
    model = _mlp()
    lam = 1e-2
    opt = IFKFAC(model, lr=1e-3, damping=lam, factor_update_freq=1)
    X = torch.randn(40, 8, generator=torch.Generator().manual_seed(9))
    acts, grads, hs = _capture(model, X)
    opt.zero_grad()
    model(X).pow(2).mean().backward()
    for h in hs:
        h.remove()
    be.cqr_status2 = 1          # the first CholeskyQR2 call reports status 2
    opt.step()
    assert be.calls["fold_finalize_cqr"] == 4      # both sides of both layers
    assert be.calls["fold_finalize"] == 5          # ... and one panel-path retry
    for m in opt.hooks.linear_layers:
        R_X, R_G = opt._factors[m]
        assert np.abs(R_X.double().numpy() - O.chol_factor([acts[m].double().numpy()], 40, lam)).max() < 1e-5
        assert np.abs(R_G.double().numpy() - O.chol_factor([grads[m].double().numpy()], 40, lam)).max() < 1e-5


def test_chunks_fold_eagerly_between_updates(be):
    """factor_update_freq = 3: steps 1 and 2 fold their chunks at once, the chunk
    of step 3 is held for the fused update; get_factors() folds a held chunk
    and leaves the running factor as an eager fold would."""
    from ifkfac_amd import IFKFAC
    model = _mlp()
    opt = IFKFAC(model, lr=1e-3, factor_update_freq=3)
    X = torch.randn(64, 8, generator=torch.Generator().manual_seed(6))
    first = opt.hooks.linear_layers[0]
    for step in (1, 2):
        opt.zero_grad()
        model(X).pow(2).mean().backward()
        assert opt.hooks._held_X[first] is None, step
        opt.step()
    opt.zero_grad()
    model(X).pow(2).mean().backward()
    assert opt.hooks._held_X[first] is not None
    f = opt.hooks.get_factors()                            # folds the held chunk
    assert opt.hooks._held_X[first] is None
    assert opt.hooks._R_X[first].shape == (8, 8) and opt.hooks._n_rows_X[first] == 3 * 64
    want = O.chol_factor([X.double().numpy()] * 3, 3 * 64, opt.damping)
    assert np.abs(f[first][0].double().numpy() - want).max() < 1e-5
    opt.step()
    assert first in opt._factors


def test_bf16_update_batches_same_shape_layers(be):
    """A consuming bf16 factor update sends the layers whose X sides and G sides
    share a shape through one batched Gram call -- one for all six sides of the
    three 12 -> 12 layers here, whose X and G sides share one signature (one
    call per side otherwise); the 12 -> 5 head's sides go alone, as batches of
    one -- every layer's factors are its own closed form, as the per-layer path
    gives them, and each side's inverse comes from the factor call (no
    separate triangular inverse)."""
    from ifkfac_amd import IFKFAC
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(12, 12), nn.Tanh(), nn.Linear(12, 12), nn.Tanh(),
                          nn.Linear(12, 12), nn.Tanh(), nn.Linear(12, 5))
    lam = 1e-2
    opt = IFKFAC(model, lr=1e-3, damping=lam, factor_update_freq=1, use_true_bf16=True)
    X = torch.randn(48, 12, generator=torch.Generator().manual_seed(3))
    acts, grads, hs = _capture(model, X)
    opt.zero_grad()
    model(X).pow(2).mean().backward()
    for h in hs:
        h.remove()
    import contextlib
    import io
    with contextlib.redirect_stdout(io.StringIO()):
        opt.step()
    # the square layers' six sides in one call, and the head's two sides
    assert be.calls["fold_finalize_gram_batched"] == be.calls["fold_finalize_gram_inverse"] == 3
    assert be.calls["fold_finalize_gram"] == 2 * 3 + 2      # six batched entries + the head
    assert be.calls["tri_inverse_bf16"] == 0
    for m in opt._factors:
        R_X, R_G = opt._factors[m]
        want_X = O.chol_factor([acts[m].double().numpy()], 48, lam)
        want_G = O.chol_factor([grads[m].double().numpy()], 48, lam)
        assert np.abs(R_X.double().numpy() - want_X).max() <= 4e-3 * np.abs(want_X).max()
        assert np.abs(R_G.double().numpy() - want_G).max() <= 4e-3 * np.abs(want_G).max()
        # the fused inverse is that of the unrounded factor; a side whose kappa
        # bound exceeds 1.5 is inverted again in fp32 from the stored bf16 factor
        fused = max(opt._kappas[m]) <= 1.5
        for Z, R, want in ((opt._inverses[m][0], R_X, want_X), (opt._inverses[m][1], R_G, want_G)):
            ref = np.linalg.inv(want if fused else R.double().numpy())
            assert np.abs(Z.double().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    assert len(opt._factors) == 4


# ---------------------------------------------------------------------------
# Classic K-FAC control (kfac_hooks.py / classic_kfac.py)
# ---------------------------------------------------------------------------
def test_kfac_hooks_average_grams_over_passes(be):
    """KFACHooks: A = sum x^T x / rows and G = sum delta^T delta / rows over every
    captured pass (kfac_hooks.py:208-266); clear() starts a new window."""
    from ifkfac_amd import KFACHooks
    model = _mlp()
    hooks = KFACHooks(model)
    hooks.enable()
    xs, ds = {m: [] for m in hooks.linear_layers}, {m: [] for m in hooks.linear_layers}
    g = torch.Generator().manual_seed(5)
    for rows in (32, 48):
        X = torch.randn(rows, 8, generator=g)
        acts, grads, hs = _capture(model, X)
        model(X).pow(2).mean().backward()
        for h in hs:
            h.remove()
        for m in hooks.linear_layers:
            xs[m].append(acts[m].double().numpy())
            ds[m].append(grads[m].double().numpy())
    f = hooks.get_factors()
    assert hooks.n_samples_accumulated() == 80
    for m in hooks.linear_layers:
        A, G = f[m]
        assert np.allclose(A.double().numpy(), O.gram_average(xs[m]), rtol=1e-5, atol=1e-6)
        assert np.allclose(G.double().numpy(), O.gram_average(ds[m]), rtol=1e-5, atol=1e-9)
    hooks.clear()
    assert hooks.get_factors() == {} and hooks.n_samples_accumulated() == 0
    hooks.remove()


def test_kfac_hooks_max_gram_dim_and_capture(be):
    from ifkfac_amd import KFACHooks
    model = nn.Sequential(nn.Linear(8, 16), nn.ReLU(), nn.Linear(16, 40))
    hooks = KFACHooks(model, max_gram_dim=32)
    assert hooks.linear_layers == [model[0]]
    hooks.enable()
    hooks.pause()
    model(torch.randn(4, 8)).sum().backward()
    assert hooks.get_factors() == {}
    with hooks.capture():
        model(torch.randn(4, 8)).sum().backward()
    assert set(hooks.get_factors()) == {model[0]}


@pytest.mark.parametrize("freq,gamma", [(1, 0.0), (3, 0.0), (1, 0.5)])
def test_classic_kfac_matches_closed_form(be, freq, gamma):
    """ClassicKFAC over 5 steps against the restated reference: the schedule
    (step % freq == 1), the Gram averages of the window, the EMA blend, damped
    inverses, G^-1 g A^-1, momentum and decoupled decay, the bias through G^-1
    without momentum, and plain SGD before the first inverses."""
    from ifkfac_amd import ClassicKFAC
    model = _mlp(seed=3)
    lr, lam, mu, wd = 1e-2, 1e-2, 0.9, 0.01
    opt = ClassicKFAC(model, lr=lr, damping=lam, factor_update_freq=freq, decomp_update_freq=freq,
                      momentum=mu, weight_decay=wd, gamma=gamma)
    layers = opt.hooks.linear_layers
    W = {m: m.weight.detach().double().numpy().copy() for m in layers}
    b = {m: m.bias.detach().double().numpy().copy() for m in layers}
    buf = {m: None for m in layers}
    window = {m: ([], []) for m in layers}
    facs, invs = {}, {}
    g = torch.Generator().manual_seed(9)
    for step in range(1, 6):
        X = torch.randn(64, 8, generator=g)
        acts, grads, hs = _capture(model, X)
        opt.zero_grad()
        model(X).pow(2).mean().backward()
        for h in hs:
            h.remove()
        gW = {m: m.weight.grad.double().numpy() for m in layers}
        gb = {m: m.bias.grad.double().numpy() for m in layers}
        opt.step()
        for m in layers:
            window[m][0].append(acts[m].double().numpy())
            window[m][1].append(grads[m].double().numpy())
        if O.classic_updates_at(step, freq):
            for m in layers:
                A, G = O.gram_average(window[m][0]), O.gram_average(window[m][1])
                if gamma > 0 and m in facs:
                    A = gamma * facs[m][0] + (1 - gamma) * A
                    G = gamma * facs[m][1] + (1 - gamma) * G
                facs[m] = (A, G)
                window[m] = ([], [])
                invs[m] = (O.classic_inverse(A, lam), O.classic_inverse(G, lam))
        for m in layers:
            if m not in invs:
                W[m] = W[m] * (1 - lr * wd) - lr * gW[m]
                b[m] = b[m] * (1 - lr * wd) - lr * gb[m]
                continue
            nat = O.classic_nat(gW[m], *invs[m])
            buf[m] = nat if buf[m] is None else mu * buf[m] + nat
            W[m] = W[m] * (1 - lr * wd) - lr * buf[m]
            b[m] = b[m] * (1 - lr * wd) - lr * (invs[m][1] @ gb[m])
        # every seam hands fp32 values on (factors, inverses, natural gradients):
        # fp32 accuracy relative to the weights' scale
        for m in layers:
            tw = 1e-5 * max(1.0, np.abs(W[m]).max())
            tb = 1e-5 * max(1.0, np.abs(b[m]).max())
            assert np.abs(m.weight.detach().double().numpy() - W[m]).max() < tw, step
            assert np.abs(m.bias.detach().double().numpy() - b[m]).max() < tb, step
    assert be.calls["gram_accumulate"] == 5 * 2 * len(layers)


# ---------------------------------------------------------------------------
# Laplace consumer (laplace.py)
# ---------------------------------------------------------------------------
def test_laplace_posterior_from_ifkfac_factors(be):
    """README.md:146-171's flow: IFKFAC captures, get_factors(), factors_to_evd,
    LaplacePosterior; a seeded draw equals the restated sample on the same Xi,
    restore_map returns the MAP weights, predictive averages softmaxes."""
    from ifkfac_amd import IFKFAC, LaplacePosterior, factors_to_evd
    model = _mlp(seed=4)
    opt = IFKFAC(model, lr=0.0, damping=1e-3, factor_update_freq=1000)
    X = torch.randn(128, 8, generator=torch.Generator().manual_seed(6))
    model(X).pow(2).mean().backward()
    factors = opt.hooks.get_factors()
    evd = factors_to_evd(factors)
    for m, (R_X, R_G) in factors.items():
        U_A, d_A, U_G, d_G = evd[m]
        for R, U, d in ((R_X, U_A, d_A), (R_G, U_G, d_G)):
            Rn = R.double().numpy()
            assert np.allclose(U.double().numpy() @ np.diag(d.double().numpy()) @ U.double().numpy().T,
                               Rn.T @ Rn, rtol=1e-5, atol=1e-6)
    W0 = {m: m.weight.detach().clone() for m in factors}
    post = LaplacePosterior(model, evd, prior_precision=10.0, dataset_size=500)
    post.sample_in_place(generator=torch.Generator().manual_seed(1))
    g = torch.Generator().manual_seed(1)
    for m in factors:
        U_A, d_A, U_G, d_G = evd[m]
        xi = torch.randn(U_G.shape[0], U_A.shape[0], generator=g).double().numpy()
        sA = O.laplace_scales(d_A.double().numpy(), 500, 10.0)
        sG = O.laplace_scales(d_G.double().numpy(), 500, 10.0)
        want = O.laplace_sample(W0[m].double().numpy(), U_A.double().numpy(), sA,
                                U_G.double().numpy(), sG, xi)
        assert np.allclose(m.weight.detach().double().numpy(), want, rtol=1e-5, atol=1e-6)
    post.restore_map()
    for m in factors:
        assert torch.equal(m.weight.detach(), W0[m])
    probs = post.predictive(X[:16], n_samples=3, generator=torch.Generator().manual_seed(2))
    assert probs.shape == (16, 4) and torch.allclose(probs.sum(-1), torch.ones(16))
    for m in factors:
        assert torch.equal(m.weight.detach(), W0[m])


# ---------------------------------------------------------------------------
# the function-level mirrors of ifkfac/triangular.py
# ---------------------------------------------------------------------------
def test_triangular_mirrors_match_oracle(be):
    """Each public function of ifkfac_amd.triangular against the oracle's restatement
    of the reference function it mirrors (triangular.py:150-227, 246-307, 331-379,
    386-421, 506-544, 551-656, 659-705)."""
    from ifkfac_amd import triangular as T
    rng = np.random.default_rng(21)
    X1, X2 = rng.standard_normal((5, 12)), rng.standard_normal((30, 12))
    t = lambda a: torch.tensor(a, dtype=torch.float32)
    # streaming update: trapezoid first, then square; R^T R = sum X^T X
    R = T.streaming_tsqr_update(None, t(X1))
    assert R.shape == (5, 12)
    R = T.streaming_tsqr_update(R, t(X2))
    want = O.streaming_tsqr_update(O.streaming_tsqr_update(None, X1), X2)
    assert R.shape == (12, 12)
    assert np.allclose(R.double().numpy(), want, atol=1e-5)
    # tsqr of a tall matrix, p < n rejected
    assert np.allclose(T.tsqr(t(X2)).double().numpy(), O.streaming_tsqr_update(None, X2), atol=1e-5)
    with pytest.raises(ValueError):
        T.tsqr(t(X1))
    # batched fold over a bucket (zero running factors, zero-padded chunks)
    B = np.stack([X2, 2 * X2])
    Rb = T.batched_streaming_tsqr_update(torch.zeros(2, 12, 12), t(B))
    for i in range(2):
        assert np.allclose(Rb[i].double().numpy(), O.streaming_tsqr_update(None, B[i]), atol=1e-5)
    # finalize: R_d^T R_d = R^T R + lambda I
    Rd = T.finalize_R(R, 1e-2).double().numpy()
    Rn = R.double().numpy()
    assert np.allclose(Rd.T @ Rd, Rn.T @ Rn + 1e-2 * np.eye(12), atol=1e-5)
    # four solves, batched, bias
    R_X = O.get_factor(O.streaming_tsqr_update(None, X2), 30, 1e-2)
    R_G = O.get_factor(O.streaming_tsqr_update(None, rng.standard_normal((40, 6))), 40, 1e-2)
    g = rng.standard_normal((6, 12))
    nat = T.apply_vered(t(g), t(R_X), t(R_G))
    assert np.allclose(nat.double().numpy(), O.apply_vered(g, R_X, R_G), rtol=1e-5, atol=1e-6)
    natb = T.apply_vered_batched(t(np.stack([g, -g])), t(np.stack([R_X, R_X])),
                                 t(np.stack([R_G, R_G])))
    assert np.allclose(natb[1].double().numpy(), -O.apply_vered(g, R_X, R_G), rtol=1e-5, atol=1e-6)
    gb = rng.standard_normal(6)
    nb = T.apply_vered_bias(t(gb), t(R_G))
    assert np.allclose(nb.double().numpy(), O.apply_vered_bias(gb, R_G), rtol=1e-5, atol=1e-6)
    # bf16 branch: non-square factors give the raw gradient back (triangular.py:608-617)
    raw = t(g)
    assert T.apply_vered(raw, t(R_X[:5]).bfloat16(), t(R_G).bfloat16()) is raw
    assert T.apply_vered_bias(t(gb), t(R_G[:3]).bfloat16()).shape == (6,)


def test_bf16_fold_takes_gram_route_when_square(be):
    """bf16 arithmetic: chunks too small for a fold that pays (fewer than 2n
    rows into a partial factor, or into the square factor) are held and
    folded together once they reach it -- by the Gram route, whose refusal
    (status 2, injected) sends the rows to the panel fold -- so a chunk of n
    rows into the square factor waits for the next one; fp32 arithmetic
    folds every chunk by the panel fold as it comes.  Whatever the grouping,
    the running factor is the oracle's of the rows folded;
    ``_running_factor`` folds the rows still held."""
    from ifkfac_amd._backend import MATH_BF16, MATH_F32
    from ifkfac_amd.activation_hooks import GRAM_FOLD_TOL, RawActivationHooks
    model = nn.Sequential(nn.Linear(8, 4))
    lin = model[0]
    rng = np.random.default_rng(3)
    chunks = [rng.standard_normal((p, 8)) for p in (5, 6, 8, 8, 8)]
    chunks[3][:, 7] = chunks[3][:, 0]            # a column repeated within the chunk
    for math_, calls, folded in ((MATH_BF16, (0, 0, 1, 0, 1), (0, 0, 3, 3, 5)),
                                 (MATH_F32, (0, 0, 0, 0, 0), (1, 2, 3, 4, 5))):
        be.calls.clear()
        hooks = RawActivationHooks(model, math=math_)
        for i, c in enumerate(chunks):
            if i == 2 and math_ == MATH_BF16:
                be.gram_fold_status2 = 1          # the device reports an ill-conditioned fold
            before = be.calls["fold_gram"]
            hooks._fold("X", lin, torch.tensor(c, dtype=torch.float32))
            assert be.calls["fold_gram"] - before == calls[i], (math_, i)
            R = hooks._R_X[lin]
            k = folded[i]
            if k == 0:
                assert R is None or R.shape[0] == 0
                continue
            old = None
            for c2 in chunks[:k]:
                old = O.streaming_tsqr_update(old, c2.astype(np.float32).astype(np.float64))
            got = R.double().numpy()
            assert got.shape == old.shape
            assert np.abs(got.T @ got - old.T @ old).max() <= 1e-5 * np.abs(old.T @ old).max(), \
                (math_, i)
        hooks.remove()
    # rows held are folded by the readers of the factor
    hooks = RawActivationHooks(model, math=MATH_BF16)
    hooks._fold("X", lin, torch.tensor(chunks[0], dtype=torch.float32))
    assert hooks._R_X[lin] is None or hooks._R_X[lin].shape[0] == 0
    R = hooks._running_factor(lin, "X").double().numpy()
    want = O.streaming_tsqr_update(None, chunks[0].astype(np.float32).astype(np.float64))
    assert np.abs(R.T @ R - want.T @ want).max() <= 1e-5 * np.abs(want.T @ want).max()
    hooks.remove()
    assert be.gram_fold_status2 == 0
    # the repeated column is refused by the pivot rule itself
    P = np.vstack([O.streaming_tsqr_update(None, np.vstack(chunks[:3])), chunks[3]])
    assert O.gram_pivot_ratio(P).min() > GRAM_FOLD_TOL   # earlier rows keep it independent
    R0 = torch.zeros(8, 8)
    st = be.fold_gram_(R0, 0, torch.tensor(chunks[3], dtype=torch.float32), GRAM_FOLD_TOL)
    assert int(st.item()) == 2 and torch.count_nonzero(R0) == 0
