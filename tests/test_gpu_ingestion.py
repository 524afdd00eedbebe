"""Conv2d im2col and 3-D (KFAC-Reduce) ingestion on the GPU.

The hooks turn a Conv2d input into its im2col rows (B * L, C_in * kH * kW) and
its output gradient into (B * H_out * W_out, C_out) rows, and flatten a 3-D
sequence tensor to (B * T, d), subsampling past a row cap by torch.randperm
(ifkfac/activation_hooks.py:489-538, :592-653; ifkfac/kfac_hooks.py:156-167).
These tests run the capture on the GPU through the HIP folds and check each
factor against the closed form of the same rows, formed independently on the
CPU in fp64 (F.unfold of the recorded conv input; the recorded rows where
randperm subsampled them):
  RawActivationHooks: ||R^T R - R_o^T R_o||_F / ||R_o^T R_o||_F <= 4 kappa(R_o) eps32,
      R_o = chol(sum X^T X / rows + damping I) (oracle.chol_factor);
  KFACHooks: ||A - X^T X / rows||_F / ||X^T X / rows||_F <= 1e-5 (fp32 sums).
"""
import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from oracle import ifk_oracle as O

pytestmark = pytest.mark.gpu

EPS32 = 1.1920929e-07
DEV = "cuda"


def _gram_rel(R, Ro):
    a = R.T @ R
    b = Ro.T @ Ro
    return np.linalg.norm(a - b) / np.linalg.norm(b)


def _kappa(Ro):
    s = np.linalg.svd(Ro, compute_uv=False)
    return s[0] / s[-1]


def _im2col_np(x, conv):
    """im2col rows of a recorded conv input, by torch's CPU unfold in fp64."""
    u = F.unfold(x.double().cpu(), kernel_size=conv.kernel_size, dilation=conv.dilation,
                 padding=conv.padding, stride=conv.stride)
    B, ckk, L = u.shape
    return u.permute(0, 2, 1).reshape(B * L, ckk).numpy()


def _grad_rows_np(g):
    B, C, H, W = g.shape
    return g.double().cpu().permute(0, 2, 3, 1).reshape(B * H * W, C).numpy()


def _conv_model():
    return nn.Sequential(nn.Conv2d(3, 8, 3, padding=1), nn.ReLU(),
                         nn.Conv2d(8, 6, 3, stride=2, dilation=2, padding=2), nn.Tanh(),
                         nn.Flatten(), nn.Linear(6 * 6 * 6, 5)).to(DEV)


def _record(model, types):
    """Forward / full-backward hooks recording each tracked module's input and
    output gradient."""
    ins, gouts, hs = {}, {}, []
    for m in model.modules():
        if isinstance(m, types):
            hs.append(m.register_forward_hook(
                lambda mod, i, o: ins.setdefault(mod, []).append(i[0].detach().clone())))
            hs.append(m.register_full_backward_hook(
                lambda mod, gi, go: gouts.setdefault(mod, []).append(go[0].detach().clone())))
    return ins, gouts, hs


@pytest.mark.parametrize("math_", [0, 1])
def test_conv2d_im2col_factors_on_gpu(hip, math_):
    """Two Conv2d layers (padding, stride 2, dilation 2) over three batches, no
    subsampling: the hooks' factors are the damped closed forms of the im2col
    rows and the flattened output gradients.  fp32 arithmetic: 4 kappa eps32.
    bf16 arithmetic: against the closed form of the bf16-rounded rows (what its
    MFMA operands are), at 5e-3 -- the bf16 panel fold's 2e-3 to 4e-3, for a
    fold the Gram route refuses (the Gram route itself keeps 1e-7 to 5e-6)."""
    from ifkfac_amd import RawActivationHooks
    torch.manual_seed(0)
    model = _conv_model()
    hooks = RawActivationHooks(model, damping=1e-2, max_conv_rows=0, math=math_)
    ins, gouts, hs = _record(model, nn.Conv2d)
    hooks.enable()
    for _ in range(3):
        x = torch.randn(16, 3, 12, 12, device=DEV)
        model(x).logsumexp(-1).sum().backward()
    factors = hooks.get_factors()
    for h in hs:
        h.remove()
    convs = [m for m in model.modules() if isinstance(m, nn.Conv2d)]
    rnd = (lambda a: a) if math_ == 0 else (
        lambda a: torch.from_numpy(a).float().to(torch.bfloat16).double().numpy())
    for conv in convs:
        X = [rnd(_im2col_np(x, conv)) for x in ins[conv]]
        G = [rnd(_grad_rows_np(g)) for g in gouts[conv]]
        rows_x = sum(a.shape[0] for a in X)
        rows_g = sum(a.shape[0] for a in G)
        assert hooks._n_rows_X[conv] == rows_x and hooks._n_rows_G[conv] == rows_g
        assert X[0].shape[1] == conv.in_channels * conv.kernel_size[0] * conv.kernel_size[1]
        R_X, R_G = factors[conv]
        for R, chunks, rows in ((R_X, X, rows_x), (R_G, G, rows_g)):
            Ro = O.chol_factor(chunks, rows, 1e-2)
            err = _gram_rel(R.double().cpu().numpy(), Ro)
            bound = 4 * _kappa(Ro) * EPS32 if math_ == 0 else 5e-3
            print(f"conv {tuple(conv.weight.shape)} math {math_}: n={Ro.shape[0]} rows={rows} "
                  f"err {err:.2e} bound {bound:.2e}")
            assert err <= bound


def test_conv2d_subsampled_rows_on_gpu(hip):
    """max_conv_rows caps each batch's im2col rows by torch.randperm on the
    device (a sample of the patches, as the reference draws it): the running
    factor holds exactly the drawn rows -- recorded here by chunk_transform_X --
    at 4 kappa eps32, with max_conv_rows rows per batch."""
    from ifkfac_amd import RawActivationHooks
    torch.manual_seed(1)
    model = _conv_model()
    hooks = RawActivationHooks(model, damping=1e-2, max_conv_rows=100)
    drawn = []
    hooks.chunk_transform_X = lambda x: (drawn.append(x.detach().clone()), x)[1]
    hooks.enable()
    for _ in range(2):
        model(torch.randn(16, 3, 12, 12, device=DEV)).sum().backward()
    factors = hooks.get_factors()
    conv = model[0]
    # forward order per batch: conv0, conv1, linear -> conv0's chunks are every third
    mine = [d for d in drawn[0::3]]
    assert all(d.shape == (100, 27) for d in mine)
    assert hooks._n_rows_X[conv] == 200
    Ro = O.chol_factor([d.double().cpu().numpy() for d in mine], 200, 1e-2)
    err = _gram_rel(factors[conv][0].double().cpu().numpy(), Ro)
    assert err <= 4 * _kappa(Ro) * EPS32


@pytest.mark.parametrize("cap", [0, 150])
def test_sequence_kfac_reduce_factors_on_gpu(hip, cap):
    """A Linear layer on (B, T, d) inputs: the hooks flatten to (B T, d) rows and,
    past max_seq_rows, keep a randperm sample of them, drawn separately for the
    input and the output-gradient side (KFAC-Reduce).  Without a cap the factors
    are the closed forms of all rows; with one, of the drawn rows (recorded by
    chunk_transform_X / _G), max_seq_rows per batch; 4 kappa eps32."""
    from ifkfac_amd import RawActivationHooks
    torch.manual_seed(2)
    model = nn.Sequential(nn.Linear(24, 40), nn.GELU(), nn.Linear(40, 12)).to(DEV)
    hooks = RawActivationHooks(model, damping=1e-2, max_seq_rows=cap)
    ins, gouts, hs = _record(model, nn.Linear)
    drawn_x, drawn_g = [], []
    hooks.chunk_transform_X = lambda x: (drawn_x.append(x.detach().clone()), x)[1]
    hooks.chunk_transform_G = lambda g: (drawn_g.append(g.detach().clone()), g)[1]
    hooks.enable()
    for _ in range(3):
        model(torch.randn(6, 40, 24, device=DEV)).pow(2).mean().backward()
    factors = hooks.get_factors()
    for h in hs:
        h.remove()
    lin = model[0]
    if cap == 0:
        X = [x.reshape(-1, 24).double().cpu().numpy() for x in ins[lin]]
        G = [g.reshape(-1, 40).double().cpu().numpy() for g in gouts[lin]]
    else:
        # forward: lin0 then lin2 per batch; backward: lin2 then lin0
        X = [d.double().cpu().numpy() for d in drawn_x[0::2]]
        G = [d.double().cpu().numpy() for d in drawn_g[1::2]]
        assert all(a.shape[0] == cap for a in X + G)
    rows_x = sum(a.shape[0] for a in X)
    rows_g = sum(a.shape[0] for a in G)
    assert rows_x == (3 * 240 if cap == 0 else 3 * cap) and rows_g == rows_x
    assert hooks._n_rows_X[lin] == rows_x and hooks._n_rows_G[lin] == rows_g
    R_X, R_G = factors[lin]
    for R, chunks, rows in ((R_X, X, rows_x), (R_G, G, rows_g)):
        Ro = O.chol_factor(chunks, rows, 1e-2)
        err = _gram_rel(R.double().cpu().numpy(), Ro)
        assert err <= 4 * _kappa(Ro) * EPS32, err


def test_classic_hooks_conv_and_sequence_on_gpu(hip):
    """The Classic control's KFACHooks on the same ingestion: Conv2d im2col rows
    and a 3-D Linear input below the subsample cap, Gram averages A = X^T X / rows
    and G = delta^T delta / rows at 1e-5 of the fp64 closed form."""
    from ifkfac_amd import KFACHooks
    torch.manual_seed(3)
    model = nn.Sequential(nn.Conv2d(3, 8, 3, padding=1), nn.ReLU(), nn.Flatten(start_dim=2),
                          nn.Linear(144, 20)).to(DEV)
    hooks = KFACHooks(model)
    ins, gouts, hs = _record(model, (nn.Conv2d, nn.Linear))
    hooks.enable()
    for _ in range(2):
        model(torch.randn(8, 3, 12, 12, device=DEV)).square().mean().backward()
    A_G = hooks.get_factors()
    for h in hs:
        h.remove()
    conv, lin = model[0], model[3]
    cases = {conv: ([_im2col_np(x, conv) for x in ins[conv]],
                    [_grad_rows_np(g) for g in gouts[conv]]),
             lin: ([x.reshape(-1, 144).double().cpu().numpy() for x in ins[lin]],
                   [g.reshape(-1, 20).double().cpu().numpy() for g in gouts[lin]])}
    for m, (X, G) in cases.items():
        A, Gm = A_G[m]
        for got, chunks in ((A, X), (Gm, G)):
            rows = sum(c.shape[0] for c in chunks)
            want = sum(c.T @ c for c in chunks) / rows
            err = np.linalg.norm(got.double().cpu().numpy() - want) / np.linalg.norm(want)
            assert err <= 1e-5, (type(m).__name__, err)
