"""Classic K-FAC, the explicit-Gram control, on the MI355X kernels.

Counterpart of ``ClassicKFAC`` (ifkfac/classic_kfac.py:25-306): the same
constructor, param groups, schedule (factors at ``step % factor_update_freq
== 1``, inverses at ``step % decomp_update_freq == 1``, both every step when
the frequency is 1: classic_kfac.py:154-159), EMA of the Gram factors
(:113-120), non-finite skip (:131-132), plain SGD for layers without inverses
(:163-185) and the per-layer update: ``G^{-1} grad A^{-1}``, clip, heavy-ball
momentum, decoupled weight decay, bias through ``G^{-1}`` without momentum
(:189-247).

Where the arithmetic happens: the Gram sums come from ``KFACHooks``
(``ifk_gram_accumulate``); each inverse is ``ifk_inv_spd_damped`` -- the
Cholesky factorisation of ``A + damping I`` and its triangular inverse in
fp32, where the reference calls ``torch.linalg.inv`` (LU); for the damped SPD
matrices of K-FAC both give the inverse to fp32 accuracy times kappa(A).  The
natural gradient is ``ifk_classic_precondition`` (two fp32 MFMA products) and
the update the fused ``ifk_momentum_update``.
"""
from __future__ import annotations

import logging
import time
from collections import deque
from typing import Dict, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from ._backend import MATH_F32, get_backend
from .kfac_hooks import KFACHooks

logger = logging.getLogger(__name__)


class ClassicKFAC(torch.optim.Optimizer):
    """K-FAC with explicit Gram factors and damped inverses (the control)."""

    def __init__(
        self,
        model: nn.Module,
        lr: float = 1e-3,
        damping: float = 1e-2,
        factor_update_freq: int = 10,
        decomp_update_freq: int = 10,
        weight_decay: float = 0.0,
        momentum: float = 0.9,
        grad_clip: Optional[float] = None,
        gamma: float = 0.0,
        max_gram_dim: int = 0,
    ):
        defaults = dict(lr=lr, damping=damping, weight_decay=weight_decay, momentum=momentum)
        params = []
        for module in model.modules():
            if isinstance(module, (nn.Linear, nn.Conv2d)):
                params.append({"params": list(module.parameters())})
        super().__init__(params, defaults)

        self.model = model
        self.damping = damping
        self.factor_update_freq = factor_update_freq
        self.decomp_update_freq = decomp_update_freq
        self.grad_clip = grad_clip
        self.gamma = gamma

        self.hooks = KFACHooks(model, max_gram_dim=max_gram_dim)
        self.hooks.enable()

        self._factors: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._inverses: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._momentum_buffers: Dict[nn.Module, torch.Tensor] = {}
        self._step_count = 0

        _maxlen = 1000
        self.timing = {
            "factor_compute": deque(maxlen=_maxlen),
            "inversion": deque(maxlen=_maxlen),
            "precondition": deque(maxlen=_maxlen),
            "total_step": deque(maxlen=_maxlen),
        }

    # ------------------------------------------------------------------ factors
    def _update_factors(self):
        """The hooks' averages, EMA-blended with the previous ones when gamma > 0."""
        t0 = time.perf_counter()
        new_factors = self.hooks.get_factors()
        self.hooks.clear()
        if self.gamma > 0.0 and self._factors:
            be = get_backend()
            for module, (A_new, G_new) in new_factors.items():
                if module in self._factors:
                    A_old, G_old = self._factors[module]
                    # gamma old + (1 - gamma) new, into the fresh averages
                    new_factors[module] = tuple(
                        self._blend(be, old, new) for old, new in ((A_old, A_new), (G_old, G_new)))
        self._factors = new_factors
        self.timing["factor_compute"].append(time.perf_counter() - t0)

    def _blend(self, be, old: torch.Tensor, new: torch.Tensor) -> torch.Tensor:
        if old.dtype != torch.float32 or new.dtype != torch.float32:
            # bf16 factors: the reference's own tensor arithmetic in that dtype
            return self.gamma * old + (1.0 - self.gamma) * new
        return be.axpby(self.gamma, old, 1.0 - self.gamma, new)

    def _update_inverses(self):
        """(A + damping I)^{-1} and (G + damping I)^{-1} of every finite factor pair;
        a pair with a non-finite entry keeps its previous inverses."""
        t0 = time.perf_counter()
        be = get_backend()
        mods = list(self._factors.keys())
        if mods:
            finite = torch.stack([torch.isfinite(t).all() for m in mods
                                  for t in self._factors[m]]).view(-1, 2).cpu()
            for i, module in enumerate(mods):
                if not bool(finite[i].all()):
                    continue
                A, G = self._factors[module]
                self._inverses[module] = (be.inv_spd_damped(A, self.damping),
                                          be.inv_spd_damped(G, self.damping))
        self.timing["inversion"].append(time.perf_counter() - t0)

    # ------------------------------------------------------------------ step
    def _group_of(self, p: torch.Tensor):
        for group in self.param_groups:
            if any(p is q for q in group["params"]):
                return group["lr"], group["weight_decay"], group["momentum"]
        return None, None, None

    @staticmethod
    def _sgd(p: torch.Tensor, g: torch.Tensor, lr: float, wd: float) -> None:
        W = p.data
        if W.dtype == torch.float32 and W.is_contiguous():
            get_backend().momentum_update_(g, None, W, lr, 0.0, wd, False)
        else:
            if wd > 0:
                W.mul_(1.0 - lr * wd)
            W.add_(g, alpha=-lr)

    @torch.no_grad()
    def step(self, closure=None):
        t_total = time.perf_counter()
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._step_count += 1

        if self._step_count % self.factor_update_freq == 1 or self.factor_update_freq == 1:
            self._update_factors()
        if self._step_count % self.decomp_update_freq == 1 or self.decomp_update_freq == 1:
            if self._factors:
                self._update_inverses()

        t_precond = time.perf_counter()
        be = get_backend()
        for module in self.hooks.linear_layers:
            if module not in self._inverses:
                # no inverses yet: plain SGD with decoupled decay on every parameter
                for p in module.parameters():
                    if p.grad is None:
                        continue
                    lr, wd, _ = self._group_of(p)
                    if lr is None:
                        continue
                    self._sgd(p, p.grad, lr, wd)
                continue
            A_inv, G_inv = self._inverses[module]
            lr, wd, mom = self._group_of(module.weight)
            if lr is None:
                continue
            if module.weight.grad is not None:
                grad_w = module.weight.grad
                shape = grad_w.shape
                nat = be.classic_precondition(grad_w.reshape(shape[0], -1), A_inv, G_inv)
                if self.grad_clip is not None:
                    gnorm = nat.norm()
                    if gnorm > self.grad_clip:
                        nat = nat * (self.grad_clip / gnorm)
                nat = nat.reshape(shape)
                W = module.weight.data
                buf = None
                init = False
                if mom > 0:
                    buf = self._momentum_buffers.get(module)
                    if buf is None:
                        buf = torch.zeros_like(nat)
                        self._momentum_buffers[module] = buf
                        init = True
                if W.dtype == torch.float32 and W.is_contiguous():
                    be.momentum_update_(nat, buf, W, lr, mom if buf is not None else 0.0, wd,
                                        init)
                else:
                    if buf is not None:
                        buf.mul_(mom).add_(nat)
                        nat = buf
                    if wd > 0:
                        W.mul_(1.0 - lr * wd)
                    W.add_(nat, alpha=-lr)
            if module.bias is not None and module.bias.grad is not None:
                g_b = module.bias.grad.reshape(-1, 1).float()
                nat_b = be.gemm(G_inv, g_b, math=MATH_F32).reshape(-1)
                self._sgd(module.bias, nat_b, lr, wd)

        self.timing["precondition"].append(time.perf_counter() - t_precond)
        self.timing["total_step"].append(time.perf_counter() - t_total)
        return loss

    # ------------------------------------------------------------------ utilities
    def get_timing_stats(self) -> Dict[str, Dict[str, float]]:
        stats: Dict[str, Dict[str, float]] = {}
        for key, times in self.timing.items():
            if times:
                arr = np.array(list(times))
                stats[key] = {
                    "mean_ms": float(arr.mean() * 1000),
                    "p50_ms": float(np.percentile(arr, 50) * 1000),
                    "p99_ms": float(np.percentile(arr, 99) * 1000),
                    "total_s": float(arr.sum()),
                    "count": len(times),
                }
        return stats

    def capture(self):
        return self.hooks.capture()

    def pause_capture(self):
        self.hooks.pause()

    def resume_capture(self):
        self.hooks.resume()

    def cleanup(self):
        self.hooks.remove()
        self._factors.clear()
        self._inverses.clear()
        self._momentum_buffers.clear()

    def __repr__(self) -> str:
        return (f"ClassicKFAC(damping={self.damping}, "
                f"factor_update_freq={self.factor_update_freq}, "
                f"decomp_update_freq={self.decomp_update_freq}, gamma={self.gamma}, "
                f"n_layers={len(self.hooks.linear_layers)})")
