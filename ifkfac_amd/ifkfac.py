"""IFKFAC optimizer on the MI355X curvature kernels.

Counterpart of ``IFKFAC`` (ifkfac/ifkfac.py:78-642): same constructor, param
groups, step schedule, factor-refresh rules (skip / clear / non-finite drop /
exact EMA blend / bf16 storage), layer classification and per-layer update
(gradient clipping, heavy-ball momentum, decoupled weight decay, bias through
the G factor only).  What changes is where the arithmetic happens:

* factor refresh: ``ifk_finalize`` damps, sign-normalises and (with
  ``use_true_bf16``) rounds each factor to bf16 in one pass and reports
  finiteness on the device; one host read per refresh collects all flags;
* after each refresh the factor inverses ``Z = R^{-1}`` are formed once
  (``ifk_tri_inverse``) and every step applies the four solves as MFMA
  products with them (``ifk_precondition_apply``);
* bf16 mode runs a layer's inverses and solves in bf16 arithmetic while both
  of its factors are near-isotropic (kappa_2 estimate from
  ``ifk_cond_estimate`` at most KAPPA_BF16_MAX), and at fp32 accuracy on the
  bf16-valued factors, the reference's regime, otherwise: fp32 inverses whose
  split bf16 halves every step applies by three MFMA products per product
  (``ifk_precondition_apply_x3``);
* momentum, decay and the weight step are one fused pass
  (``ifk_momentum_update``).
"""
from __future__ import annotations

import logging
import math
import time
import warnings
from collections import deque
from typing import Dict, Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from ._backend import MATH_BF16, MATH_F32, get_backend, run_pair
from .activation_hooks import IFKFACRankError, RawActivationHooks
from .triangular import solve_math_for

logger = logging.getLogger(__name__)

# bf16 mode: a layer keeps bf16 arithmetic for its solves while both of its
# factors have kappa_2(R) <= KAPPA_BF16_MAX; otherwise its inverses and applies
# run in fp32 arithmetic on the bf16-valued factors, as the reference's bf16
# mode does (ifkfac/triangular.py:621-628).  The bf16 products' rounding is
# amplified by kappa(A) kappa(G) = kappa(R_X)^2 kappa(R_G)^2 for a gradient
# aligned with the factors' dominant directions (as a layer's gradient is):
# measured 5e-3 against fp64 solves of the same factors at kappa 1, 1.4e-2 to
# 3e-2 at kappa 3.1-3.2, while the fp32 arithmetic stays near 6e-6.
KAPPA_BF16_MAX = 1.5
# ifk_cond_estimate is a power-iteration lower bound of kappa_2 (up to about
# 10 % low); it is raised by this factor before the comparison, so that the
# gate errs towards fp32 arithmetic (the Gram route's bound is an upper bound
# and is taken as is).
COND_ESTIMATE_MARGIN = 1.1


class IFKFAC(torch.optim.Optimizer):
    """K-FAC with QR-based factors and triangular solves (no explicit Gram inverse).

    Parameters are those of the reference (ifkfac/ifkfac.py:119-136).
    """

    def __init__(
        self,
        model: nn.Module,
        lr: float = 1e-3,
        damping: float = 1e-2,
        factor_update_freq: int = 10,
        weight_decay: float = 0.0,
        momentum: float = 0.9,
        grad_clip: Optional[float] = None,
        gamma: float = 0.0,
        max_out_dim: int = 0,
        augment_bias: bool = False,
        max_conv_rows: int = 512,
        max_seq_rows: Optional[int] = None,
        batched_qr: bool = False,
        deferred_qr: bool = False,
        use_true_bf16: bool = False,
    ):
        self.use_true_bf16 = use_true_bf16
        params = []
        for module in model.modules():
            if isinstance(module, (nn.Linear, nn.Conv2d)):
                params.append({"params": list(module.parameters())})
        defaults = dict(lr=lr, weight_decay=weight_decay, momentum=momentum)
        super().__init__(params, defaults)

        self.model = model
        self.damping = damping
        self.factor_update_freq = factor_update_freq
        self.grad_clip = grad_clip
        self.gamma = gamma
        self.augment_bias = augment_bias
        self._math = MATH_BF16 if use_true_bf16 else MATH_F32

        self.hooks = RawActivationHooks(
            model,
            damping=damping,
            max_out_dim=max_out_dim,
            augment_bias=augment_bias,
            max_conv_rows=max_conv_rows,
            max_seq_rows=max_seq_rows,
            batched=batched_qr,
            deferred=deferred_qr,
            math=self._math,
        )
        self.hooks.enable()
        # the chunks captured before an update step feed a fused fold + finalize
        self.hooks._defer_last = self._updates_at(1)

        self._factors: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._inverses: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        # bf16 arithmetic: RNE bf16 copies ((Z_X, Z_X^T), (Z_G, Z_G^T)) per layer
        self._inverse_copies: Dict[nn.Module, tuple] = {}
        # fp32 accuracy: split bf16 halves (Z_hi, Z_lo, Z^T_hi, Z^T_lo) per side
        self._split_copies: Dict[nn.Module, tuple] = {}
        # per layer: MFMA arithmetic of its solves, and the kappa_2 estimates
        # (R_X, R_G) that chose it (bf16 mode)
        self._solve_math: Dict[nn.Module, int] = {}
        self._kappas: Dict[nn.Module, Tuple[float, float]] = {}
        self._classic_fallback: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._momentum_buffers: Dict[nn.Module, torch.Tensor] = {}
        self._step_count = 0

        _maxlen = 1000
        self.timing: Dict[str, deque] = {
            "factor_compute": deque(maxlen=_maxlen),
            "precondition": deque(maxlen=_maxlen),
            "total_step": deque(maxlen=_maxlen),
        }

    # ------------------------------------------------------------------ factors
    def _blend(self, R_old: torch.Tensor, R_new: torch.Tensor) -> torch.Tensor:
        """Factor of [sqrt(g) R_old; sqrt(1-g) R_new] (ifkfac/ifkfac.py:270-278)."""
        n = R_new.shape[0]
        buf = (math.sqrt(self.gamma) * R_old.float()).contiguous()
        X = (math.sqrt(1.0 - self.gamma) * R_new.float()).contiguous()
        get_backend().fold_(buf, n, X, self._math)
        return buf

    def _updates_at(self, step: int) -> bool:
        """Whether step number ``step`` (1-based) updates the factors (ifkfac.py:560-564)."""
        f = self.factor_update_freq
        return f == 1 or (step >= f and step % f == 0)

    def _update_factors(self):
        t0 = time.perf_counter()
        blend = self.gamma > 0.0 and bool(self._factors)
        out_dtype = torch.bfloat16 if (self.use_true_bf16 and not blend) else torch.float32
        be = get_backend()
        copies = hasattr(be, "tri_inverse_bf16")
        split = hasattr(be, "precondition_apply_x3")
        x3_inverse = hasattr(be, "tri_inverse_x3")
        # bf16 factors in bf16 arithmetic: the Gram route's call forms each
        # side's inverse as well
        fused_inverse = (copies and out_dtype == torch.bfloat16
                         and solve_math_for(torch.bfloat16) == MATH_BF16)

        def inverse(side, module, R, kappa_bound=None, inv=None):
            m = solve_math_for(R.dtype)
            if inv is not None and m == MATH_BF16:
                # formed by the Gram route's call from the Cholesky's 1024-block
                # inverses, with its bf16 copies
                return inv[0], inv[1], inv[2], kappa_bound
            if m == MATH_BF16 and copies:
                # bf16 arithmetic: keep the bf16 copies of Z and Z^T next to Z,
                # so the per-step apply does not cast the inverses again.  The
                # choice of arithmetic needs kappa_2(R): the Gram path's upper
                # bound when the factor came from it, else an estimate
                Z, Zb, ZT = be.tri_inverse_bf16(R)
                k = (kappa_bound if kappa_bound is not None
                     else COND_ESTIMATE_MARGIN * be.cond_estimate(R, Z))
                return Z, Zb, ZT, k
            return be.tri_inverse(R, m)

        try:
            # the hooks are cleared right after: a held chunk may be consumed.
            # Without a blend each side's inverse follows its factor on its
            # stream, so the narrower side's inverse runs while the wider one
            # is still being factored.
            new_factors, flags, early = self.hooks._collect_factors(
                out_dtype, consume=True, then=None if blend else inverse,
                with_inverse=fused_inverse)
        except IFKFACRankError as e:
            logger.warning("IFKFAC: factor update skipped — %s", e)
            self.timing["factor_compute"].append(time.perf_counter() - t0)
            return

        self.hooks.clear()

        clean: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        if new_factors:
            mods = list(new_factors.keys())
            ok = torch.cat([torch.cat(flags[m]) for m in mods]).view(-1, 2).cpu()
            for i, module in enumerate(mods):
                if not bool(ok[i].all()):
                    logger.warning("IFKFAC: non-finite R for layer %s — skipping.",
                                   type(module).__name__)
                    continue
                clean[module] = new_factors[module]

        if blend:
            blended = {}
            for module, (R_X_new, R_G_new) in clean.items():
                if module in self._factors:
                    R_X_old, R_G_old = self._factors[module]
                    blended[module] = (self._blend(R_X_old, R_X_new),
                                       self._blend(R_G_old, R_G_new))
                else:
                    blended[module] = (R_X_new, R_G_new)
            clean = blended
            if self.use_true_bf16:
                clean = {m: (a.to(torch.bfloat16), b.to(torch.bfloat16))
                         for m, (a, b) in clean.items()}

        self._factors = clean
        self._inverses = {}
        self._inverse_copies = {}
        self._split_copies = {}
        self._solve_math = {}
        self._kappas = {}
        invs = {}
        for module, (R_X, R_G) in clean.items():
            if early is not None:
                invs[module] = early[module]
            else:
                invs[module] = run_pair(R_X.device, lambda R=R_X: inverse("X", module, R),
                                        lambda R=R_G: inverse("G", module, R),
                                        b_first=R_G.shape[0] > R_X.shape[0])
        # one host read of every kappa estimate (the flags were read above)
        bf = [m for m, (iX, _) in invs.items() if isinstance(iX, tuple)]
        kap = torch.cat([torch.cat([invs[m][0][3], invs[m][1][3]]) for m in bf]).view(-1, 2).cpu() \
            if bf else None
        fp32_solves = []
        for module, (invX, invG) in invs.items():
            R_X, R_G = clean[module]
            if not isinstance(invX, tuple):
                self._inverses[module] = (invX, invG)
                self._solve_math[module] = solve_math_for(R_X.dtype)
                continue
            kx, kg = (float(v) for v in kap[bf.index(module)])
            self._kappas[module] = (kx, kg)
            if kx <= KAPPA_BF16_MAX and kg <= KAPPA_BF16_MAX:
                self._inverses[module] = (invX[0], invG[0])
                self._inverse_copies[module] = ((invX[1], invX[2]), (invG[1], invG[2]))
                self._solve_math[module] = MATH_BF16
            else:
                # fp32 accuracy on the bf16-valued factors (the reference's
                # regime): inverses at fp32 accuracy -- from split bf16
                # halves on the wide levels when the backend has them, the
                # same accuracy class as the apply -- applied through their
                # split bf16 halves (three MFMA products per solve product)
                # when the backend has that apply, else by fp32 arithmetic
                logger.debug("IFKFAC: kappa(R_X) %.3g, kappa(R_G) %.3g: fp32 solves for %s",
                             kx, kg, type(module).__name__)
                inv32 = ((lambda R: be.tri_inverse_x3(R)) if split and x3_inverse
                         else (lambda R: be.tri_inverse(R, MATH_F32)))
                ZX, ZG = run_pair(R_X.device, lambda R=R_X: inv32(R), lambda R=R_G: inv32(R),
                                  b_first=R_G.shape[0] > R_X.shape[0])
                self._inverses[module] = (ZX, ZG)
                self._solve_math[module] = MATH_F32
                fp32_solves.append(module)
        if split and fp32_solves:
            # the split halves of same-shape layers in one buffer per side, at
            # one stride from layer to layer, so their apply can be grouped
            groups: Dict[tuple, list] = {}
            for module in fp32_solves:
                ZX, ZG = self._inverses[module]
                groups.setdefault((ZX.shape[0], ZG.shape[0], ZX.device), []).append(module)
            batched = hasattr(be, "inverse_split_copies_batched")
            for mods in groups.values():
                if batched and len(mods) > 1:
                    sxs = be.inverse_split_copies_batched([self._inverses[m][0] for m in mods])
                    sgs = be.inverse_split_copies_batched([self._inverses[m][1] for m in mods])
                else:
                    sxs = [be.inverse_split_copies(self._inverses[m][0]) for m in mods]
                    sgs = [be.inverse_split_copies(self._inverses[m][1]) for m in mods]
                for m, sx, sg in zip(mods, sxs, sgs):
                    self._split_copies[m] = (sx, sg)
        self.timing["factor_compute"].append(time.perf_counter() - t0)

    # ------------------------------------------------------------------ apply
    def _get_module_hp(self, module):
        for group in self.param_groups:
            if any(p is module.weight for p in group["params"]):
                return group["lr"], group["weight_decay"], group["momentum"]
        return None, None, None

    def _nat_grad(self, module: nn.Module, grad_w: torch.Tensor, trim: bool) -> torch.Tensor:
        copies = self._inverse_copies.get(module)
        if copies is not None:
            (ZXb, ZXt), ZG2 = copies
            if trim:
                ZXb, ZXt = ZXb[:-1, :-1], ZXt[:-1, :-1]
            return get_backend().precondition_apply_bf16(grad_w, (ZXb, ZXt), ZG2)
        split = self._split_copies.get(module)
        if split is not None:
            sx, sg = split
            if trim:
                sx = tuple(t[:-1, :-1] for t in sx)
            return get_backend().precondition_apply_x3(grad_w, sx, sg)
        Z_X, Z_G = self._inverses[module]
        if trim:
            Z_X = Z_X[:-1, :-1]
        R_X = self._factors[module][0]
        m = self._solve_math.get(module, solve_math_for(R_X.dtype))
        return get_backend().precondition_apply(grad_w, Z_X, Z_G, m)

    def _nat_grads_grouped(self, mods) -> list:
        """_nat_grad for a bucket of same-shape layers (apply_vered_batched,
        ifkfac/triangular.py:506-544): the layers that take the same apply and
        whose inverse copies sit at one stride from layer to layer (as the
        batched factor update and inverse_split_copies_batched leave them) go
        through one grouped call, each product one launch over the group; the
        others layer by layer.  Every layer gets the bits its own call gives."""
        be = get_backend()
        out = {}
        bf = [m for m in mods if m in self._inverse_copies]
        x3 = [m for m in mods if m not in self._inverse_copies and m in self._split_copies]
        if len(bf) > 1 and hasattr(be, "precondition_apply_bf16_batched"):
            ZX2s = [self._inverse_copies[m][0] for m in bf]
            ZG2s = [self._inverse_copies[m][1] for m in bf]
            if all(be.entry_stride(list(ts)) is not None
                   for side in (ZX2s, ZG2s) for ts in zip(*side)):
                nat = be.precondition_apply_bf16_batched([m.weight.grad for m in bf], ZX2s, ZG2s)
                out.update({m: nat[e] for e, m in enumerate(bf)})
        if len(x3) > 1 and hasattr(be, "precondition_apply_x3_batched"):
            sxs = [self._split_copies[m][0] for m in x3]
            sgs = [self._split_copies[m][1] for m in x3]
            if all(be.entry_stride(list(ts)) is not None
                   for side in (sxs, sgs) for ts in zip(*side)):
                nat = be.precondition_apply_x3_batched([m.weight.grad for m in x3], sxs, sgs)
                out.update({m: nat[e] for e, m in enumerate(x3)})
        return [out[m] if m in out else self._nat_grad(m, m.weight.grad, False) for m in mods]

    def _update_param(self, param: torch.Tensor, nat: torch.Tensor, lr: float, wd: float,
                      mom: float, module: Optional[nn.Module], clip: bool = False) -> None:
        """Clip (``clip`` and grad_clip set), momentum (module given and mom > 0),
        decay, step.  Only a weight's natural gradient is clipped
        (ifkfac/ifkfac.py:397-400, 494-497); bias updates (:418-423, :515-519)
        and the plain-SGD step of a layer without factors (:443-448) are not."""
        if clip and self.grad_clip is not None:
            gnorm = nat.norm()
            if gnorm > self.grad_clip:
                nat = nat * (self.grad_clip / gnorm)
        buf = None
        init = False
        if module is not None and mom > 0:
            buf = self._momentum_buffers.get(module)
            if buf is None:
                buf = torch.zeros_like(param.data, dtype=torch.float32)
                self._momentum_buffers[module] = buf
                init = True
        W = param.data
        if W.dtype == torch.float32 and W.is_contiguous():
            get_backend().momentum_update_(nat, buf, W, lr, mom if buf is not None else 0.0, wd,
                                           init)
        else:
            # non-fp32 or strided parameters: the reference's own tensor ops
            nat = nat.reshape(W.shape)
            if buf is not None:
                buf.mul_(mom).add_(nat)
                nat = buf
            if wd > 0:
                W.mul_(1.0 - lr * wd)
            # one rounding to W's dtype, as torch's in-place add does for the
            # reference's fp32 natural gradient (ifkfac/ifkfac.py:413)
            W.add_(nat, alpha=-lr)

    def _update_bias(self, module: nn.Module, lr: float, wd: float) -> None:
        if module.bias is None or module.bias.grad is None:
            return
        Z_G = self._inverses[module][1]
        nat_b = get_backend().precondition_bias(module.bias.grad, Z_G)
        self._update_param(module.bias, nat_b, lr, wd, 0.0, None)

    def _apply_preconditioner_bucketed(self):
        fast: Dict[tuple, list] = {}
        slow_modules = []
        for module in self.hooks.linear_layers:
            if module.weight.grad is None:
                continue
            lr, wd, mom = self._get_module_hp(module)
            if lr is None:
                continue
            if module not in self._factors:
                slow_modules.append((module, lr, wd, mom))
                continue
            R_X, R_G = self._factors[module]
            weight = module.weight
            is_linear_2d = isinstance(module, nn.Linear) and weight.dim() == 2
            needs_trim = self.augment_bias and module.bias is not None
            if not is_linear_2d or needs_trim:
                slow_modules.append((module, lr, wd, mom))
                continue
            key = (R_X.shape[0], R_G.shape[0], weight.dtype, weight.device)
            fast.setdefault(key, []).append((module, lr, wd, mom))

        for module, lr, wd, mom in slow_modules:
            self._apply_preconditioner(module, lr=lr, weight_decay=wd, momentum=mom)

        for (n_in, n_out, _, _), entries in fast.items():
            try:
                nats = self._nat_grads_grouped([m for m, _, _, _ in entries])
            except Exception as e:  # same recovery as the reference's bucket failure
                logger.warning(
                    "IFKFAC: apply_vered_batched failed for bucket (n_in=%d, n_out=%d, B=%d): "
                    "%s — falling back to per-layer.", n_in, n_out, len(entries), e)
                for m, lr, wd, mom in entries:
                    self._apply_preconditioner(m, lr=lr, weight_decay=wd, momentum=mom)
                continue
            for (m, lr, wd, mom), nat in zip(entries, nats):
                self._update_param(m.weight, nat, lr, wd, mom, m, clip=True)
                self._update_bias(m, lr, wd)

    def _apply_preconditioner(self, module: nn.Module, lr: float, weight_decay: float,
                              momentum: float):
        weight = module.weight
        if weight.grad is None:
            return
        if module not in self._factors:
            # plain SGD with decoupled decay; bias untouched (ifkfac/ifkfac.py:443-448)
            self._update_param(weight, weight.grad, lr, weight_decay, 0.0, None)
            return
        grad_w = weight.grad
        trim = self.augment_bias and module.bias is not None
        orig_shape = grad_w.shape
        if grad_w.dim() > 2:
            grad_w = grad_w.reshape(orig_shape[0], -1)
        try:
            nat = self._nat_grad(module, grad_w, trim)
        except Exception as e:
            logger.warning("IFKFAC: apply_vered failed for %s (%s) — using raw gradient.",
                           type(module).__name__, e)
            nat = grad_w
        nat = nat.reshape(orig_shape)
        self._update_param(weight, nat, lr, weight_decay, momentum, module, clip=True)
        self._update_bias(module, lr, weight_decay)

    # ------------------------------------------------------------------ step
    @torch.no_grad()
    def step(self, closure=None):
        t_total = time.perf_counter()
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        self._step_count += 1
        _verbose = self._step_count <= 20
        if _verbose:
            print(f"    [IFKFAC step={self._step_count}] entry", flush=True)
        self.hooks.flush()
        if _verbose:
            print(f"    [IFKFAC step={self._step_count}] hooks.flush done", flush=True)

        if self.factor_update_freq == 1:
            self._update_factors()
        elif (self._step_count >= self.factor_update_freq
              and self._step_count % self.factor_update_freq == 0):
            self._update_factors()
        self.hooks._defer_last = self._updates_at(self._step_count + 1)

        t_precond = time.perf_counter()
        self._apply_preconditioner_bucketed()
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
        self._inverse_copies.clear()
        self._split_copies.clear()
        self._solve_math.clear()
        self._kappas.clear()
        self._classic_fallback.clear()
        self._momentum_buffers.clear()

    def __repr__(self) -> str:
        return (f"IFKFAC(damping={self.damping}, factor_update_freq={self.factor_update_freq}, "
                f"gamma={self.gamma}, augment_bias={self.augment_bias}, "
                f"n_layers={len(self.hooks.linear_layers)})")
