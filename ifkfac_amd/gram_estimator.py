"""Hook-estimator interface shared by the factor-capture classes.

Mirrors ``GramMatrixEstimator`` (ifkfac/gram_estimator.py:28-173): the abstract
lifecycle (enable / get_factors / clear / remove / linear_layers) and the
capture controls ``pause``, ``resume`` and the ``capture`` context manager,
which toggle a writeable ``_enabled`` flag that the hooks test before doing
any work.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from contextlib import contextmanager
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn


class GramMatrixEstimator(ABC):
    """Abstract base of per-layer curvature-factor estimators."""

    @abstractmethod
    def enable(self) -> None:
        """Attach forward and backward hooks to all tracked layers."""

    @abstractmethod
    def get_factors(self) -> Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]]:
        """Return the per-layer factor pair for every layer with data."""

    @abstractmethod
    def clear(self) -> None:
        """Reset the accumulators (start a new window)."""

    @abstractmethod
    def remove(self) -> None:
        """Detach all hooks and free the accumulated state."""

    @property
    @abstractmethod
    def linear_layers(self) -> List[nn.Module]:
        """Tracked ``nn.Linear`` / ``nn.Conv2d`` modules, in model order."""

    def n_samples_accumulated(self, module: Optional[nn.Module] = None) -> int:
        """Rows accumulated since the last ``clear()`` (0 unless overridden)."""
        return 0

    @property
    def is_enabled(self) -> bool:
        return False

    # capture controls (ifkfac/gram_estimator.py:137-173)
    def pause(self) -> None:
        """Keep the hooks attached but make them no-ops."""
        self._enabled = False

    def resume(self) -> None:
        """Undo :meth:`pause`."""
        self._enabled = True

    @contextmanager
    def capture(self):
        """Enable capture inside the ``with`` block; restore the old state after."""
        previous = getattr(self, "_enabled", False)
        self._enabled = True
        try:
            yield self
        finally:
            self._enabled = previous
