"""ifkfac_amd -- the IFKFAC curvature path on MI355X (gfx950) HIP kernels.

Drop-in for the reference package's optimizer-facing API (ifkfac/__init__.py:23-35):

    from ifkfac_amd import IFKFAC
    opt = IFKFAC(model, lr=1e-3, damping=1e-2, factor_update_freq=1, momentum=0.9,
                 use_true_bf16=True)
    loss.backward(); opt.step()
    factors = opt.hooks.get_factors()

All curvature arithmetic runs in ``libifkfac_hip.so`` (include/ifkfac_hip.h);
tensors must live on a ROCm device.
"""
from .activation_hooks import IFKFACRankError, RawActivationHooks
from .classic_kfac import ClassicKFAC
from .ifkfac import IFKFAC
from .kfac_hooks import KFACHooks
from .laplace import LaplacePosterior, factors_to_evd
from ._lib import IFKFACBackendError

__version__ = "0.1.0"
__all__ = [
    "IFKFAC",
    "ClassicKFAC",
    "KFACHooks",
    "LaplacePosterior",
    "factors_to_evd",
    "RawActivationHooks",
    "IFKFACRankError",
    "IFKFACBackendError",
]
