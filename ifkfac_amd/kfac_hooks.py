"""Gram-matrix factor capture for the Classic K-FAC control.

Counterpart of ``KFACHooks`` (ifkfac/kfac_hooks.py:61-297): forward and
backward hooks on every ``nn.Linear`` / ``nn.Conv2d`` (optionally skipping
layers whose output dimension exceeds ``max_gram_dim``) accumulate running
sums ``A_sum += x^T x`` and ``G_sum += delta^T delta`` with their row counts,
and ``get_factors()`` returns the averages ``(A_sum / n_A, G_sum / n_G)``.
Conv2d inputs are unfolded (im2col) and their output gradients flattened to
``(B*H_out*W_out, C_out)``; 3-D sequence tensors are flattened and, beyond
``_SEQ_SUBSAMPLE`` rows, subsampled by ``torch.randperm`` (KFAC-Reduce), as in
the reference.

The arithmetic runs in the HIP library: each hook's contribution is one
``ifk_gram_accumulate`` (lower-triangle MFMA product in the activations' own
arithmetic, mirrored, added into the fp32 sum in the same pass) and the
averages are one ``ifk_axpby``.  The sums are held in fp32 whatever the
activation dtype; ``get_factors()`` returns the averages in the dtype of the
layer's last captured input (the reference keeps bf16 sums for bf16
activations: its values differ from these by that rounding).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from ._backend import get_backend
from .activation_hooks import RawActivationHooks
from .gram_estimator import GramMatrixEstimator


class KFACHooks(GramMatrixEstimator):
    """Running Gram sums of every tracked layer's inputs and output gradients."""

    # rows kept from a flattened 3-D input (kfac_hooks.py:156-167)
    _SEQ_SUBSAMPLE: int = 2048

    def __init__(self, model: nn.Module, max_gram_dim: int = 0):
        self.model = model
        self.max_gram_dim = max_gram_dim
        self._handles: List[torch.utils.hooks.RemovableHandle] = []
        self._A_sum: Dict[nn.Module, torch.Tensor] = {}
        self._G_sum: Dict[nn.Module, torch.Tensor] = {}
        self._n_A: Dict[nn.Module, int] = {}
        self._n_G: Dict[nn.Module, int] = {}
        self._dtype: Dict[nn.Module, torch.dtype] = {}
        self._enabled = False
        self._linear_layers: List[nn.Module] = []
        for module in model.modules():
            if isinstance(module, (nn.Linear, nn.Conv2d)):
                if max_gram_dim > 0:
                    out_dim = (module.out_features if isinstance(module, nn.Linear)
                               else module.out_channels)
                    if out_dim > max_gram_dim:
                        continue
                self._linear_layers.append(module)

    @property
    def linear_layers(self) -> List[nn.Module]:
        return self._linear_layers

    @property
    def is_enabled(self) -> bool:
        return self._enabled

    def enable(self):
        if self._enabled:
            return
        for module in self._linear_layers:
            self._handles.append(module.register_forward_hook(self._forward_hook))
            self._handles.append(module.register_full_backward_hook(self._backward_hook))
        self._enabled = True

    # the im2col / flattening of the IFKFAC hooks: the same transforms
    # (kfac_hooks.py:126-145 = activation_hooks.py:489-508)
    _unfold_conv_input = staticmethod(RawActivationHooks._unfold_conv_input)
    _reshape_conv_grad = staticmethod(RawActivationHooks._reshape_conv_grad)

    def _rows(self, t: torch.Tensor) -> torch.Tensor:
        t = t.reshape(-1, t.shape[-1])
        if t.shape[0] > self._SEQ_SUBSAMPLE:
            idx = torch.randperm(t.shape[0], device=t.device)[: self._SEQ_SUBSAMPLE]
            t = t[idx]
        return t

    def _accumulate(self, sums: Dict[nn.Module, torch.Tensor], counts: Dict[nn.Module, int],
                    module: nn.Module, rows: torch.Tensor) -> None:
        n = rows.shape[1]
        S = sums.get(module)
        first = S is None
        if first:
            S = torch.empty((n, n), dtype=torch.float32, device=rows.device)
            sums[module] = S
        get_backend().gram_accumulate_(S, rows, 0.0 if first else 1.0)
        counts[module] = (0 if first else counts[module]) + rows.shape[0]

    def _forward_hook(self, module: nn.Module, input: Tuple[torch.Tensor, ...],
                      output: torch.Tensor):
        """A_sum += x^T x (kfac_hooks.py:169-214)."""
        if not self._enabled:
            return
        x = input[0].detach()
        if isinstance(module, nn.Conv2d):
            x = self._unfold_conv_input(x, module)
        elif x.ndim > 2:
            x = self._rows(x)
        self._dtype[module] = x.dtype
        self._accumulate(self._A_sum, self._n_A, module, x)

    def _backward_hook(self, module: nn.Module, grad_input: Tuple[torch.Tensor, ...],
                       grad_output: Tuple[torch.Tensor, ...]):
        """G_sum += delta^T delta (kfac_hooks.py:216-245)."""
        if not self._enabled:
            return
        delta = grad_output[0].detach()
        if isinstance(module, nn.Conv2d):
            delta = self._reshape_conv_grad(delta)
        elif delta.ndim > 2:
            delta = self._rows(delta)
        self._accumulate(self._G_sum, self._n_G, module, delta)

    def get_factors(self) -> Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]]:
        """(A_sum / n_A, G_sum / n_G) of every layer with both sums (kfac_hooks.py:247-266)."""
        be = get_backend()
        factors: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        for module in self._linear_layers:
            if module not in self._A_sum or module not in self._G_sum:
                continue
            A = be.axpby(1.0 / self._n_A[module], self._A_sum[module], 0.0)
            G = be.axpby(1.0 / self._n_G[module], self._G_sum[module], 0.0)
            dt = self._dtype.get(module, torch.float32)
            if dt != torch.float32:
                A, G = A.to(dt), G.to(dt)
            factors[module] = (A, G)
        return factors

    def n_samples_accumulated(self, module: Optional[nn.Module] = None) -> int:
        target = module or (self._linear_layers[0] if self._linear_layers else None)
        if target is None:
            return 0
        return self._n_A.get(target, 0)

    def clear(self):
        self._A_sum.clear()
        self._G_sum.clear()
        self._n_A.clear()
        self._n_G.clear()

    def remove(self):
        for h in self._handles:
            h.remove()
        self._handles.clear()
        self._enabled = False
        self.clear()
