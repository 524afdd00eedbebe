"""Grouped launches for same-shape layers (the reference's bucketed apply and
flush: ifkfac/triangular.py:331-379, 506-544; ifkfac/activation_hooks.py:370-457;
ifkfac/ifkfac.py:371-380).

Each grouped call runs every product once over the group and must give every
layer exactly the bits of its own per-layer call (torch.equal), for the bf16
apply, the split (x3) apply, and the Gram-route streaming fold of a flush,
including an entry the Gram route refuses.  End to end, IFKFAC's bucketed
apply and RawActivationHooks' batched flush with the grouped calls give the
same weights and factors as with the grouped calls hidden from them.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _upper_inverse(n, g, scale=1.0):
    R = torch.triu(torch.randn(n, n, device=DEV, generator=g)) * 0.05 * scale
    R += torch.eye(n, device=DEV)
    return torch.linalg.inv(R.double()).float().triu().contiguous()


@pytest.mark.parametrize("n_out,n_in", [(1024, 1024), (1536, 512)])
def test_apply_bf16_batched_bit_equal(hip, n_out, n_in):
    """B = 4 layers: the bf16 apply from copies stacked in one (B, n, n) buffer
    per side against the per-layer ifk_precondition_apply_bf16."""
    g = torch.Generator(device=DEV).manual_seed(n_out + n_in)
    B = 4
    ZX = torch.stack([_upper_inverse(n_in, g) for _ in range(B)])
    ZG = torch.stack([_upper_inverse(n_out, g) for _ in range(B)])
    ZXb, ZXt = ZX.bfloat16(), ZX.transpose(1, 2).contiguous().bfloat16()
    ZGb, ZGt = ZG.bfloat16(), ZG.transpose(1, 2).contiguous().bfloat16()
    grads = [torch.randn(n_out, n_in, device=DEV, generator=g) * 0.1 for _ in range(B)]
    nat = hip.precondition_apply_bf16_batched(grads, [(ZXb[e], ZXt[e]) for e in range(B)],
                                              [(ZGb[e], ZGt[e]) for e in range(B)])
    for e in range(B):
        one = hip.precondition_apply_bf16(grads[e], (ZXb[e], ZXt[e]), (ZGb[e], ZGt[e]))
        assert torch.equal(nat[e], one), e


@pytest.mark.parametrize("n_out,n_in", [(1024, 1024), (512, 1536)])
def test_apply_x3_batched_bit_equal(hip, n_out, n_in):
    """B = 3 layers: the split apply from halves made by
    inverse_split_copies_batched against the per-layer ifk_precondition_apply_x3
    on the per-layer halves (which are bit-equal too)."""
    g = torch.Generator(device=DEV).manual_seed(7 + n_out)
    B = 3
    ZXs = [_upper_inverse(n_in, g, 3.0) for _ in range(B)]
    ZGs = [_upper_inverse(n_out, g, 3.0) for _ in range(B)]
    sx = hip.inverse_split_copies_batched(ZXs)
    sg = hip.inverse_split_copies_batched(ZGs)
    grads = [torch.randn(n_out, n_in, device=DEV, generator=g) * 0.1 for _ in range(B)]
    nat = hip.precondition_apply_x3_batched(grads, sx, sg)
    for e in range(B):
        sx1, sg1 = hip.inverse_split_copies(ZXs[e]), hip.inverse_split_copies(ZGs[e])
        assert all(torch.equal(a, b) for a, b in zip(sx[e], sx1))
        one = hip.precondition_apply_x3(grads[e], sx1, sg1)
        assert torch.equal(nat[e], one), e


@pytest.mark.parametrize("n,p", [(768, 4096), (2304, 4096)])
def test_fold_gram_batched_bit_equal(hip, n, p):
    """B = 4 running factors of one shape, each folding its own chunk: the
    batched Gram-route fold against the per-layer fold_gram_, factors and
    statuses bit-equal; entry 2's chunk repeats a column of large scale, so the
    Gram route refuses it (status 2) and its buffer stays untouched."""
    from ifkfac_amd.activation_hooks import GRAM_FOLD_TOL
    g = torch.Generator(device=DEV).manual_seed(n)
    B = 4
    Rs0 = []
    for e in range(B):
        R = torch.zeros(n, n, device=DEV)
        assert hip.fold_gram_(R, 0, torch.randn(p, n, device=DEV, generator=g),
                              GRAM_FOLD_TOL).item() == 1
        Rs0.append(R)
    Xs = [torch.randn(p, n, device=DEV, generator=g) for _ in range(B)]
    Xs[2][:, 5] *= 1e3
    Xs[2][:, 17] = Xs[2][:, 5]
    Rb = [R.clone() for R in Rs0]
    st = hip.fold_gram_batched_(Rb, n, Xs, GRAM_FOLD_TOL)
    for e in range(B):
        R1 = Rs0[e].clone()
        s1 = hip.fold_gram_(R1, n, Xs[e], GRAM_FOLD_TOL)
        assert int(st[e].item()) == int(s1.item())
        assert torch.equal(Rb[e], R1), e
    assert int(st[2].item()) == 2 and torch.equal(Rb[2], Rs0[2])
    assert all(int(st[e].item()) == 1 for e in (0, 1, 3))


class _Hide:
    """Hide attributes of the backend object for the duration (the callers take
    the per-layer path when a grouped method is missing)."""

    def __init__(self, be, names):
        self.be, self.names, self.saved = be, names, {}

    def __enter__(self):
        cls = type(self.be)
        for nm in self.names:
            self.saved[nm] = getattr(cls, nm)
            delattr(cls, nm)

    def __exit__(self, *a):
        cls = type(self.be)
        for nm, f in self.saved.items():
            setattr(cls, nm, f)


def _mlp(seed, n=1024, layers=4):
    torch.manual_seed(seed)
    mods = []
    for _ in range(layers):
        mods += [nn.Linear(n, n), nn.GELU()]
    return nn.Sequential(*mods).to(DEV)


def test_ifkfac_grouped_apply_matches_per_layer(hip):
    """4 x (Linear(1024, 1024) + GELU), bf16 factors: the first layer's input is
    near-isotropic (bf16 apply), the GELU inputs are not (split apply), so the
    bucket holds a group of each kind.  Two optimizer steps with the grouped
    applies give bit for bit the weights of the same steps with the grouped
    methods hidden, and the grouped calls were made."""
    from ifkfac_amd import IFKFAC
    import contextlib, io
    calls = {"bf16": 0, "x3": 0}
    cls = type(hip)
    real_b, real_x = cls.precondition_apply_bf16_batched, cls.precondition_apply_x3_batched

    def wrap_b(self, *a):
        calls["bf16"] += 1
        return real_b(self, *a)

    def wrap_x(self, *a):
        calls["x3"] += 1
        return real_x(self, *a)

    def run(grouped):
        model = _mlp(0)
        opt = IFKFAC(model, lr=1e-2, damping=1e-2, factor_update_freq=1, momentum=0.9,
                     use_true_bf16=True)
        g = torch.Generator(device=DEV).manual_seed(1)
        x = torch.randn(2048, 1024, device=DEV, generator=g)
        tgt = torch.randn(2048, 1024, device=DEV, generator=g) * 0.1
        for _ in range(2):
            opt.zero_grad()
            ((model(x) - tgt) ** 2).mean().backward()
            with contextlib.redirect_stdout(io.StringIO()):
                opt.step()
        torch.cuda.synchronize()
        return [p.detach().clone() for p in model.parameters()], opt

    cls.precondition_apply_bf16_batched, cls.precondition_apply_x3_batched = wrap_b, wrap_x
    try:
        Wg, opt = run(True)
    finally:
        cls.precondition_apply_bf16_batched, cls.precondition_apply_x3_batched = real_b, real_x
    modes = ["bf16" if m in opt._inverse_copies else "x3" for m in opt._factors]
    print(f"apply modes {modes}; grouped calls {calls}")
    with _Hide(hip, ["precondition_apply_bf16_batched", "precondition_apply_x3_batched",
                     "inverse_split_copies_batched"]):
        Wp, _ = run(False)
    assert sum(c > 0 for c in calls.values()) >= 1
    if modes.count("x3") > 1:
        assert calls["x3"] == 2
    for a, b in zip(Wg, Wp):
        assert torch.equal(a, b)


def test_hooks_batched_flush_grouped_matches_per_layer(hip):
    """RawActivationHooks(batched=True) in bf16 arithmetic over three same-shape
    layers: the flush folds each side's buffered chunks of the three layers by
    one batched Gram-route fold; the factors are bit for bit those of the
    per-layer flush."""
    from ifkfac_amd import RawActivationHooks
    from ifkfac_amd._backend import MATH_BF16

    def run():
        model = _mlp(3, n=768, layers=3)
        hooks = RawActivationHooks(model, damping=1e-3, batched=True, math=MATH_BF16)
        hooks.enable()
        g = torch.Generator(device=DEV).manual_seed(4)
        for _ in range(2):
            x = torch.randn(1024, 768, device=DEV, generator=g)
            model(x).square().mean().backward()
            hooks.flush()
        f = hooks.get_factors()
        return [tuple(t.clone() for t in f[m]) for m in model if isinstance(m, nn.Linear)]

    grouped = run()
    with _Hide(hip, ["fold_gram_batched_"]):
        single = run()
    for a, b in zip(grouped, single):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_hooks_grouped_folds_match_per_layer(hip):
    """RawActivationHooks (per-batch folds) in bf16 arithmetic over three
    same-shape layers, 2048-row batches: each batch's Gram-route folds of the
    three layers are held and go through one batched fold per side (the first
    batch's trapezoid folds included); after three batches the factors are bit
    for bit those of the per-layer folds, and the batched fold was called."""
    from ifkfac_amd import RawActivationHooks
    from ifkfac_amd._backend import MATH_BF16
    calls = [0]
    cls = type(hip)
    real = cls.fold_gram_batched_

    def wrap(self, *a):
        calls[0] += 1
        return real(self, *a)

    def run():
        model = _mlp(5, n=768, layers=3)
        hooks = RawActivationHooks(model, damping=1e-3, math=MATH_BF16)
        hooks.enable()
        g = torch.Generator(device=DEV).manual_seed(6)
        for _ in range(3):
            x = torch.randn(2048, 768, device=DEV, generator=g)
            model(x).square().mean().backward()
        f = hooks.get_factors()
        return [tuple(t.clone() for t in f[m]) for m in model if isinstance(m, nn.Linear)]

    cls.fold_gram_batched_ = wrap
    try:
        grouped = run()
    finally:
        cls.fold_gram_batched_ = real
    with _Hide(hip, ["fold_gram_batched_"]):
        single = run()
    print(f"batched folds {calls[0]}")
    assert calls[0] >= 2
    for a, b in zip(grouped, single):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_fold_groups_merge_narrower_square_group(hip):
    """FoldGroups.flush with square factors of widths 2304 and 3072 (4096-row
    chunks, a ViT-B block's qkv and fc1/fc2 sides): the 2304-wide entries ride
    the 3072-wide group's batched fold embedded as [[R, 0], [0, I]], so one
    batched call takes all of them; every factor is that of its rows (the
    chunk's bf16 rounding, the running factor to fp32 accuracy) within 1e-4,
    and a 2304-wide entry the Gram route refuses (a repeated column at 1e3
    times the others' scale) is folded by the panel path once its status is
    read, its factor untouched by the merged fold."""
    from ifkfac_amd.activation_hooks import FoldGroups, FoldStatusQueue
    from ifkfac_amd._backend import MATH_BF16
    from oracle import ifk_oracle as O
    rng = np.random.default_rng(11)
    t = lambda a: torch.tensor(a, dtype=torch.float32, device=DEV)
    widths = [2304, 3072, 3072, 2304]
    Rs, chunks, R0 = [], [], []
    for n in widths:
        R = t(O.streaming_tsqr_update(None, rng.standard_normal((n + 512, n)) * 0.5))
        Rs.append(R)
        R0.append(R.double().cpu().numpy())
        chunks.append(rng.standard_normal((4096, n)))
    chunks[3][:, 7] *= 1e3
    chunks[3][:, 11] = chunks[3][:, 7]
    calls = []
    cls = type(hip)
    real = cls.fold_gram_batched_

    def wrap(self, Rs_, r_in, Xs, tol):
        calls.append((len(Rs_), r_in, Xs[0].shape[1]))
        return real(self, Rs_, r_in, Xs, tol)

    q = FoldStatusQueue()
    g = FoldGroups()
    for i, (R, X) in enumerate(zip(Rs, chunks)):
        g.hold(i, R, R.shape[0], t(X))
    cls.fold_gram_batched_ = wrap
    try:
        g.flush(MATH_BF16, q)
    finally:
        cls.fold_gram_batched_ = real
    q.drain()
    print(f"batched calls {calls}, refused {q.refused}")
    assert calls == [(4, 3072, 3072)]
    assert q.refused == 1
    for i, n in enumerate(widths):
        got = Rs[i].double().cpu().numpy()
        if i == 3:
            ref = O.streaming_tsqr_update(R0[i], chunks[i])
            tol = 4 * np.linalg.cond(ref) * 1.1920929e-07
        else:
            rows = O.bf16_round(chunks[i].astype(np.float32)).astype(np.float64)
            ref = O.streaming_tsqr_update(R0[i], rows)
            tol = 1e-4
        a, w = got.T @ got, ref.T @ ref
        e = np.linalg.norm(a - w) / np.linalg.norm(w)
        print(f"entry {i} n={n}: {e:.2e}")
        assert e <= tol, (i, e)


def test_get_factors_grouped_by_width(hip):
    """get_factors() in bf16 arithmetic (the Laplace use, no factor update):
    the running factors of every layer and side go through one batched
    Gram-route finalize per width -- widths 384 (five sides), 1536 (two) and
    1152, which rides the 1536 group embedded as [[R, 0], [0, I]] -- with the
    factors of the per-side finalizes: bit for bit where the width has its
    own group, within 1e-5 (relative Gram error of the damped factor) where it
    rides a wider one."""
    from ifkfac_amd import RawActivationHooks
    from ifkfac_amd._backend import MATH_BF16
    calls = []
    cls = type(hip)
    real = cls.fold_finalize_gram_batched

    def wrap(self, Rs, r_in, Xs, *a, **k):
        calls.append((len(Xs), Xs[0].shape[1]))
        return real(self, Rs, r_in, Xs, *a, **k)

    def run():
        torch.manual_seed(8)
        layers = nn.ModuleList([nn.Linear(384, 1152), nn.Linear(384, 384), nn.Linear(384, 1536),
                                nn.Linear(1536, 384)]).to(DEV)
        hooks = RawActivationHooks(layers, damping=1e-3, math=MATH_BF16)
        hooks.enable()
        g = torch.Generator(device=DEV).manual_seed(9)
        for _ in range(2):
            x = torch.randn(2048, 384, device=DEV, generator=g)
            h = layers[0](x)[:, :384] + layers[1](x) + layers[3](torch.tanh(layers[2](x)))
            h.square().mean().backward()
            layers.zero_grad()
        f = hooks.get_factors()
        return [tuple(t.clone() for t in f[m]) for m in layers]

    cls.fold_finalize_gram_batched = wrap
    try:
        grouped = run()
    finally:
        cls.fold_finalize_gram_batched = real
    print(f"batched finalize calls {sorted(calls)}")
    assert sorted(calls) == [(2 + 1, 1536), (5, 384)]
    with _Hide(hip, ["fold_finalize_gram_batched"]):
        single = run()
    for li, (a, b) in enumerate(zip(grouped, single)):
        for side, (x, y) in enumerate(zip(a, b)):
            if x.shape[0] == 1152:
                xd, yd = x.double(), y.double()
                e = float((xd.t() @ xd - yd.t() @ yd).norm() / (yd.t() @ yd).norm())
                assert e <= 1e-5, (li, side, e)
            else:
                assert torch.equal(x, y), (li, side)
