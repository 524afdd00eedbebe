"""K-FAC Laplace posterior fed by the IFKFAC factors, on the MI355X kernels.

Counterpart of ``ifkfac/laplace.py`` (``LaplacePosterior``, :61-226) plus the
``factors_to_evd`` helper its README uses (README.md:146-171) but the
reference never defines.  Per layer the posterior covariance is the Kronecker
product of ``U diag(1 / (sqrt(N) d + sqrt(lambda))) U^T`` over the two sides,
with ``(U, d)`` the eigendecomposition of the side's Gram factor, and a weight
sample is ``W_map + U_G diag(s_G) Xi diag(s_A) U_A^T`` with
``s = 1 / sqrt(sqrt(N) d + sqrt(lambda))`` and ``Xi ~ N(0, 1)`` (laplace.py:
84-101, :138-154).

``factors_to_evd`` takes the factors of ``hooks.get_factors()`` (upper
triangular R with ``R^T R = A``) and returns ``(U_A, d_A, U_G, d_G)`` with
``A = U_A diag(d_A) U_A^T``: the right singular vectors and squared singular
values of R, computed from R itself (``ifk_factor_evd``: one-sided block
Jacobi), never from the formed ``R^T R``, so the small eigenvalues keep the
relative accuracy kappa(R) allows rather than kappa(R)^2 -- the property
laplace.py:26-30 attributes to ``svd(R)``.  Eigenvalues come out descending,
as ``torch.linalg.svd`` orders singular values.

Sampling draws ``Xi`` with ``torch.randn`` exactly as the reference does (same
shape, dtype, device and generator, so a seeded generator gives the same
draws) and forms the sample in one ``ifk_laplace_sample`` call (row/column
scaling and two fp32 MFMA products into the weight).
"""
from __future__ import annotations

import logging
import time
from typing import Dict, Optional, Tuple

import torch
import torch.nn as nn

from ._backend import get_backend

logger = logging.getLogger(__name__)


def _sync(t: torch.Tensor) -> None:
    if t.is_cuda:
        torch.cuda.synchronize(t.device)


# (U_A, d_A, U_G, d_G): eigenvectors (columns) and eigenvalues of A and G
EVDFactor = Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]


def factors_to_evd(factors: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]]
                   ) -> Dict[nn.Module, EVDFactor]:
    """``{module: (R_X, R_G)}`` -> ``{module: (U_A, d_A, U_G, d_G)}`` with
    ``R_X^T R_X = U_A diag(d_A) U_A^T`` and likewise for G (fp32, d descending)."""
    be = get_backend()
    out: Dict[nn.Module, EVDFactor] = {}
    sweeps = []
    for module, (R_X, R_G) in factors.items():
        U_A, d_A, sw_a = be.factor_evd(R_X)
        U_G, d_G, sw_g = be.factor_evd(R_G)
        out[module] = (U_A, d_A, U_G, d_G)
        sweeps += [sw_a, sw_g]
    if sweeps:
        s = torch.cat(sweeps).cpu()
        if bool((s <= 0).any()):
            logger.warning("factors_to_evd: %d factor(s) did not reach the Jacobi tolerance",
                           int((s <= 0).sum()))
    return out


class LaplacePosterior:
    """K-FAC Laplace posterior (Daxberger et al. 2021, section 4 and appendix A).

    Parameters are those of the reference (laplace.py:79-85): the trained
    ``model`` at its MAP weights, ``factors_evd`` from :func:`factors_to_evd`,
    ``prior_precision`` (lambda) and ``dataset_size`` (N).
    """

    # the reference times each layer of the first sampling call (laplace.py:71-72)
    _diag_first_call: bool = True

    def __init__(self, model: nn.Module, factors_evd: Dict[nn.Module, EVDFactor],
                 prior_precision: float = 1.0, dataset_size: int = 1):
        self.model = model
        self.prior_precision = prior_precision
        self.dataset_size = dataset_size
        self._w_map: Dict[nn.Module, torch.Tensor] = {
            mod: mod.weight.data.clone() for mod in factors_evd}
        be = get_backend()
        sqrt_n = float(dataset_size) ** 0.5
        sqrt_lam = float(prior_precision) ** 0.5
        self._factors: Dict[nn.Module, EVDFactor] = {}
        for mod, (U_A, d_A, U_G, d_G) in factors_evd.items():
            self._factors[mod] = (
                U_A.to(torch.float32).contiguous(),
                be.laplace_scales(d_A, sqrt_n, sqrt_lam),
                U_G.to(torch.float32).contiguous(),
                be.laplace_scales(d_G, sqrt_n, sqrt_lam),
            )

    @torch.no_grad()
    def sample_in_place(self, generator: Optional[torch.Generator] = None):
        """Overwrite every layer with factors by one posterior draw around its MAP
        weight (laplace.py:112-158); other layers keep their values."""
        be = get_backend()
        timed = LaplacePosterior._diag_first_call
        for mod, (U_A, s_A, U_G, s_G) in self._factors.items():
            if timed:
                _sync(mod.weight)
                t0 = time.perf_counter()
            n_in, n_out = U_A.shape[0], U_G.shape[0]
            W = mod.weight.data
            xi = torch.randn(n_out, n_in, device=W.device, dtype=torch.float32,
                             generator=generator)
            w_map = self._w_map[mod]
            if W.dtype == torch.float32 and W.is_contiguous() and w_map.is_contiguous():
                be.laplace_sample_(w_map.view(n_out, n_in), W.view(n_out, n_in), U_G, s_G, U_A,
                                   s_A, xi)
            else:
                # other weight dtypes: the fp32 perturbation, rounded once into W
                delta = torch.zeros((n_out, n_in), dtype=torch.float32, device=W.device)
                be.laplace_sample_(delta, delta, U_G, s_G, U_A, s_A, xi)
                W.copy_(w_map)
                W.add_(delta.reshape(W.shape).to(W.dtype))
            if timed:
                _sync(mod.weight)
                logger.info("sample_in_place: %s n_in=%d n_out=%d %.2f ms", type(mod).__name__,
                            n_in, n_out, 1e3 * (time.perf_counter() - t0))
        if timed:
            LaplacePosterior._diag_first_call = False

    @torch.no_grad()
    def restore_map(self):
        """Reset the weights to the MAP point."""
        for mod in self._factors:
            mod.weight.data.copy_(self._w_map[mod])

    @torch.no_grad()
    def predictive(self, x: torch.Tensor, n_samples: int = 30,
                   generator: Optional[torch.Generator] = None) -> torch.Tensor:
        """Monte-Carlo predictive class probabilities of one batch (laplace.py:166-186)."""
        was_training = self.model.training
        self.model.eval()
        probs_sum = None
        for _ in range(n_samples):
            self.sample_in_place(generator=generator)
            p = torch.softmax(self.model(x).float(), dim=-1)
            probs_sum = p if probs_sum is None else probs_sum + p
        self.restore_map()
        if was_training:
            self.model.train()
        return probs_sum / n_samples

    @torch.no_grad()
    def predictive_full_loader(self, loader, device, n_samples: int = 30,
                               generator: Optional[torch.Generator] = None
                               ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Predictive over a whole loader, one weight draw per pass over it
        (laplace.py:188-226): (probabilities (N, classes), labels (N,))."""
        was_training = self.model.training
        self.model.eval()
        probs_sum = None
        labels_all = None
        for _ in range(n_samples):
            self.sample_in_place(generator=generator)
            batch_probs, batch_labels = [], []
            for x, y in loader:
                x = x.to(device, non_blocking=True)
                batch_probs.append(torch.softmax(self.model(x).float(), dim=-1).cpu())
                if labels_all is None:
                    batch_labels.append(y)
            probs = torch.cat(batch_probs)
            probs_sum = probs if probs_sum is None else probs_sum + probs
            if labels_all is None:
                labels_all = torch.cat(batch_labels)
        self.restore_map()
        if was_training:
            self.model.train()
        return probs_sum / n_samples, labels_all
