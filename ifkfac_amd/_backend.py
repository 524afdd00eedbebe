"""Tensor-level dispatch of the curvature path into the HIP library.

Every function here takes torch tensors that live on a ROCm device, passes
raw device pointers, sizes and the caller's current stream through the C ABI,
and allocates outputs and workspaces with torch's caching allocator.  There
is no second implementation: CPU tensors, a missing library or a failed call
raise.

``get_backend()`` returns the process-wide backend (the HIP one unless a test
installed a double with ``set_backend``).
"""
from __future__ import annotations

import ctypes
import math as _math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import IFK_BF16, IFK_F32, IFK_MATH_BF16, IFK_MATH_F32, IFKFACBackendError

MATH_F32 = IFK_MATH_F32
MATH_BF16 = IFK_MATH_BF16
# Relative pivot threshold of the Gram route's factor update (status 2 below
# it: the side is refactored by the panel path); the library's default too.
GRAM_PIVOT_TOL = 1e-3

_DT = {torch.float32: IFK_F32, torch.bfloat16: IFK_BF16}
_TORCH_DT = {IFK_F32: torch.float32, IFK_BF16: torch.bfloat16}


def _require_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise IFKFACBackendError(
            f"{what}: tensor is on {t.device}; the IFKFAC curvature kernels run only on a "
            "ROCm GPU")


def _mat(t: torch.Tensor, what: str) -> Tuple[torch.Tensor, int, int]:
    """Return (t', ld, dtype code) with t' 2-D, row-major rows, fp32 or bf16."""
    _require_device(t, what)
    if t.dim() != 2:
        raise IFKFACBackendError(f"{what}: expected a 2-D tensor, got shape {tuple(t.shape)}")
    if t.dtype not in _DT:
        t = t.float()
    if t.stride(1) != 1 or (t.shape[0] > 1 and t.stride(0) < t.shape[1]):
        t = t.contiguous()
    ld = t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)
    return t, ld, _DT[t.dtype]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


class HipBackend:
    """Dispatch to libifkfac_hip.so."""

    name = "hip"

    def __init__(self) -> None:
        self.lib = _lib.load()

    # -- plumbing --------------------------------------------------------------
    @staticmethod
    def _stream(dev: torch.device) -> int:
        return torch.cuda.current_stream(dev).cuda_stream

    @staticmethod
    def _ws(nbytes: int, dev: torch.device) -> torch.Tensor:
        return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)

    # -- streaming TSQR fold ---------------------------------------------------
    def fold_(self, R: torch.Tensor, r_in: int, X: torch.Tensor, math: int) -> int:
        """Fold chunk X (p x n) into R (n x n fp32 buffer, rows [0, r_in) valid) in place."""
        _require_device(R, "tsqr_fold")
        n = R.shape[1]
        if R.dtype != torch.float32 or R.shape[0] != n or not R.is_contiguous():
            raise IFKFACBackendError("tsqr_fold: R must be a contiguous n x n fp32 buffer")
        X, ldx, xdt = _mat(X, "tsqr_fold")
        if X.shape[1] != n:
            raise IFKFACBackendError(f"tsqr_fold: chunk has {X.shape[1]} columns, R has {n}")
        p = X.shape[0]
        ws = self._ws(self.lib.ifk_tsqr_fold_workspace_size(p, n), R.device)
        r_out = _lib.ctypes.c_int64(0)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_tsqr_fold(self._stream(R.device), _ptr(X), xdt, p, n, ldx, _ptr(R), n,
                                        int(r_in), int(math), _ptr(ws), ws.numel(),
                                        _lib.ctypes.byref(r_out))
        _lib.check(rc, "ifk_tsqr_fold")
        return int(r_out.value)

    def fold_gram_(self, R: torch.Tensor, r_in: int, X: torch.Tensor,
                   pivot_tol: float) -> torch.Tensor:
        """Fold chunk X into R by the Gram route (bf16 arithmetic, r_in + p >= n).

        Returns the device int32[1] status: 1 R holds the factor of
        [R[:r_in]; X] (n rows); 2 a pivot fell below ``pivot_tol`` of its Gram
        diagonal or the input is not finite -- R is then unchanged and the
        caller folds by ``fold_``.
        """
        _require_device(R, "tsqr_fold_gram")
        n = R.shape[1]
        if R.dtype != torch.float32 or R.shape[0] != n or not R.is_contiguous():
            raise IFKFACBackendError("tsqr_fold_gram: R must be a contiguous n x n fp32 buffer")
        X, ldx, xdt = _mat(X, "tsqr_fold_gram")
        if X.shape[1] != n:
            raise IFKFACBackendError(f"tsqr_fold_gram: chunk has {X.shape[1]} columns, R has {n}")
        p = X.shape[0]
        st = torch.empty(1, dtype=torch.int32, device=R.device)
        ws = self._ws(self.lib.ifk_tsqr_fold_gram_workspace_size(p, n, int(r_in)), R.device)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_tsqr_fold_gram(self._stream(R.device), _ptr(X), xdt, p, n, ldx,
                                             _ptr(R), n, int(r_in), float(pivot_tol), _ptr(st),
                                             _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_tsqr_fold_gram")
        return st

    # -- damping / finalisation -------------------------------------------------
    def finalize(self, R: torch.Tensor, scale: float, damping: float, out_dtype: torch.dtype,
                 math: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Return (R_damped, finite flag int32[1]) for a square R."""
        R, ldr, rdt = _mat(R, "finalize")
        if rdt != IFK_F32:
            R = R.float()
            ldr = R.stride(0)
        n = R.shape[1]
        if R.shape[0] != n:
            raise IFKFACBackendError("finalize: R must be square")
        out = torch.empty((n, n), dtype=out_dtype, device=R.device)
        flag = torch.empty(1, dtype=torch.int32, device=R.device)
        ws = self._ws(self.lib.ifk_finalize_workspace_size(n), R.device)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_finalize(self._stream(R.device), _ptr(R), ldr, n, float(scale),
                                       float(damping), _ptr(out), _DT[out_dtype], n, int(math),
                                       _ptr(flag), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_finalize")
        return out, flag

    def fold_finalize(self, R: Optional[torch.Tensor], r_in: int, X: torch.Tensor, scale: float,
                      damping: float, out_dtype: torch.dtype, math: int,
                      cqr: bool = False, gram: bool = False, with_kappa: bool = False):
        """finalize(fold(R[:r_in], X)) in one factorisation, leaving R untouched.

        Returns (R_damped, finite flag int32[1]); R (n x n fp32 buffer whose
        first r_in rows are the running factor) may be None when r_in == 0.
        With ``cqr`` the outer blocks are factored by CholeskyQR2
        (ifk_fold_finalize_cqr); with ``gram`` (bf16 arithmetic only) the
        factor is the Cholesky factor of the Gram matrix
        (ifk_fold_finalize_gram).  Either way the flag is then 1 / 0 as
        above, or 2 when the input was too ill-conditioned for that method --
        the caller must then call again with neither.  With ``with_kappa``
        (Gram path) a third value is returned: a device float[1] upper bound
        of kappa_2 of the factor.
        """
        X, ldx, xdt = _mat(X, "fold_finalize")
        p, n = X.shape
        ldr = n
        if r_in > 0:
            if R is None or R.dtype != torch.float32 or R.shape[1] != n or R.shape[0] < r_in:
                raise IFKFACBackendError("fold_finalize: R must be an fp32 buffer with n columns "
                                         "and at least r_in rows")
            _require_device(R, "fold_finalize")
            if R.stride(1) != 1:
                R = R.contiguous()
            ldr = R.stride(0) if R.shape[0] > 1 else n
        out = torch.empty((n, n), dtype=out_dtype, device=X.device)
        flag = torch.empty(1, dtype=torch.int32, device=X.device)
        kb = torch.empty(1, dtype=torch.float32, device=X.device) if (gram and with_kappa) else None
        if gram and math != MATH_BF16:
            raise IFKFACBackendError("fold_finalize: the Gram path is bf16 arithmetic only")
        name = ("ifk_fold_finalize_gram" if gram else
                "ifk_fold_finalize_cqr" if cqr else "ifk_fold_finalize")
        ws = self._ws(getattr(self.lib, name + "_workspace_size")(p, n, int(r_in)), X.device)
        extra = (_ptr(kb),) if gram else ()
        with torch.cuda.device(X.device):
            rc = getattr(self.lib, name)(self._stream(X.device), _ptr(X), xdt, p, n, ldx,
                                         _ptr(R) if r_in > 0 else None, ldr, int(r_in),
                                         float(scale), float(damping), _ptr(out),
                                         _DT[out_dtype], n, int(math), _ptr(flag), *extra,
                                         _ptr(ws), ws.numel())
        _lib.check(rc, name)
        return (out, flag, kb) if kb is not None else (out, flag)

    def status_to_host(self, st: torch.Tensor, host: torch.Tensor) -> None:
        """host[:n] <- st[:n] (int32; host pinned) by a kernel on the current
        stream (ifk_status_to_host); read it after an event recorded behind."""
        _require_device(st, "status_to_host")
        if (st.dtype != torch.int32 or host.dtype != torch.int32 or not host.is_pinned()
                or host.numel() < st.numel() or not st.is_contiguous()):
            raise IFKFACBackendError("status_to_host: int32 device status, pinned int32 host")
        with torch.cuda.device(st.device):
            rc = self.lib.ifk_status_to_host(self._stream(st.device), _ptr(st), host.data_ptr(),
                                             st.numel())
        _lib.check(rc, "ifk_status_to_host")

    def fold_gram_batched_(self, Rs, r_in: int, Xs, pivot_tol: float) -> torch.Tensor:
        """fold_gram_ for B running factors of one shape, each folding its own
        chunk, in one chain of launches (ifk_tsqr_fold_gram_batched).  Rs:
        contiguous n x n fp32 buffers; Xs: B chunks (p x n, one dtype).
        Returns the device int32[B] statuses; entry e's R and status are bitwise
        what fold_gram_ gives it alone (R untouched where the status is 2)."""
        B = len(Xs)
        mats = [_mat(X, "tsqr_fold_gram_batched") for X in Xs]
        X0, ldx, xdt = mats[0]
        p, n = X0.shape
        if any(m[0].shape != (p, n) or m[1] != ldx or m[2] != xdt for m in mats):
            raise IFKFACBackendError("tsqr_fold_gram_batched: chunks differ in shape or dtype")
        for R in Rs:
            _require_device(R, "tsqr_fold_gram_batched")
            if R.dtype != torch.float32 or R.shape != (n, n) or not R.is_contiguous():
                raise IFKFACBackendError("tsqr_fold_gram_batched: each R must be a contiguous "
                                         "n x n fp32 buffer")
        dev = X0.device
        xptrs = (ctypes.c_void_p * B)(*[m[0].data_ptr() for m in mats])
        rptrs = (ctypes.c_void_p * B)(*[R.data_ptr() for R in Rs])
        st = torch.empty(B, dtype=torch.int32, device=dev)
        ws = self._ws(self.lib.ifk_tsqr_fold_gram_batched_workspace_size(B, p, n, int(r_in)),
                      dev)
        with torch.cuda.device(dev):
            rc = self.lib.ifk_tsqr_fold_gram_batched(
                self._stream(dev), B, ctypes.cast(xptrs, ctypes.c_void_p), xdt, p, n, ldx,
                ctypes.cast(rptrs, ctypes.c_void_p), n, int(r_in), float(pivot_tol), _ptr(st),
                _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_tsqr_fold_gram_batched")
        return st

    def fold_finalize_gram_batched(self, Rs, r_in: int, Xs, scale: float, damping: float,
                                   out_dtype: torch.dtype, with_inverse: bool = False,
                                   pivot_tol: float = GRAM_PIVOT_TOL):
        """fold_finalize(..., gram=True, with_kappa=True) for B same-shape sides in
        the same launches (ifk_fold_finalize_gram_batched).  Xs: B chunks (p x n,
        one dtype); Rs: B running-factor buffers or None when r_in == 0.
        Returns (factors (B, n, n), status int32[B], kappa bound float32[B]); entry
        b is bitwise the single-side result.  With ``with_inverse``
        (ifk_fold_finalize_gram_inverse) a fourth value (Z fp32, Zb, ZT bf16, each
        (B, n, n)): each factor's inverse and its bf16 copies, from the Cholesky's
        1024-block inverses (meaningless where the status is 2).  ``pivot_tol``: the
        relative pivot threshold of the status."""
        B = len(Xs)
        mats = [_mat(X, "fold_finalize_gram_batched") for X in Xs]
        X0, ldx, xdt = mats[0]
        p, n = X0.shape
        if any(m[0].shape != (p, n) or m[1] != ldx or m[2] != xdt for m in mats):
            raise IFKFACBackendError("fold_finalize_gram_batched: chunks differ in shape or dtype")
        ldr = n
        rptrs = None
        if r_in > 0:
            Rs = [R if R.stride(1) == 1 else R.contiguous() for R in Rs]
            for R in Rs:
                if R.dtype != torch.float32 or R.shape[1] != n or R.shape[0] < r_in:
                    raise IFKFACBackendError("fold_finalize_gram_batched: bad running factor")
                _require_device(R, "fold_finalize_gram_batched")
            ldr = Rs[0].stride(0) if Rs[0].shape[0] > 1 else n
            if any((R.stride(0) if R.shape[0] > 1 else n) != ldr for R in Rs):
                raise IFKFACBackendError("fold_finalize_gram_batched: running factors differ "
                                         "in row stride")
            rptrs = (ctypes.c_void_p * B)(*[R.data_ptr() for R in Rs])
        xptrs = (ctypes.c_void_p * B)(*[m[0].data_ptr() for m in mats])
        dev = X0.device
        out = torch.empty((B, n, n), dtype=out_dtype, device=dev)
        st = torch.empty(B, dtype=torch.int32, device=dev)
        kb = torch.empty(B, dtype=torch.float32, device=dev)
        if with_inverse:
            Z = torch.empty((B, n, n), dtype=torch.float32, device=dev)
            Zb = torch.empty((B, n, n), dtype=torch.bfloat16, device=dev)
            ZT = torch.empty((B, n, n), dtype=torch.bfloat16, device=dev)
            ws = self._ws(self.lib.ifk_fold_finalize_gram_inverse_workspace_size(
                B, p, n, int(r_in)), dev)
            with torch.cuda.device(dev):
                rc = self.lib.ifk_fold_finalize_gram_inverse(
                    self._stream(dev), B, ctypes.cast(xptrs, ctypes.c_void_p), xdt, p, n, ldx,
                    ctypes.cast(rptrs, ctypes.c_void_p) if rptrs is not None else None, ldr,
                    int(r_in), float(scale), float(damping), _ptr(out), _DT[out_dtype], n, n * n,
                    float(pivot_tol), _ptr(st), _ptr(kb), _ptr(Z), n, n * n, _ptr(Zb), _ptr(ZT),
                    n, n * n,
                    _ptr(ws), ws.numel())
            _lib.check(rc, "ifk_fold_finalize_gram_inverse")
            return out, st, kb, (Z, Zb, ZT)
        ws = self._ws(self.lib.ifk_fold_finalize_gram_batched_workspace_size(B, p, n, int(r_in)),
                      dev)
        with torch.cuda.device(dev):
            rc = self.lib.ifk_fold_finalize_gram_batched(
                self._stream(dev), B, ctypes.cast(xptrs, ctypes.c_void_p), xdt, p, n, ldx,
                ctypes.cast(rptrs, ctypes.c_void_p) if rptrs is not None else None, ldr,
                int(r_in), float(scale), float(damping), _ptr(out), _DT[out_dtype], n, n * n,
                MATH_BF16, float(pivot_tol), _ptr(st), _ptr(kb), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_fold_finalize_gram_batched")
        return out, st, kb

    # -- preconditioning ------------------------------------------------------------
    def tri_inverse(self, R: torch.Tensor, math: int) -> torch.Tensor:
        R, ldr, rdt = _mat(R, "tri_inverse")
        n = R.shape[0]
        if R.shape[1] != n:
            raise IFKFACBackendError("tri_inverse: R must be square")
        Z = torch.empty((n, n), dtype=torch.float32, device=R.device)
        ws = self._ws(self.lib.ifk_tri_inverse_workspace_size(n), R.device)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_tri_inverse(self._stream(R.device), _ptr(R), rdt, ldr, n, _ptr(Z), n,
                                          int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_tri_inverse")
        return Z

    def tri_inverse_x3(self, R: torch.Tensor) -> torch.Tensor:
        """tri_inverse at about fp32 accuracy on bf16 MFMA (split halves on
        the wide levels; ifk_tri_inverse_x3)."""
        R, ldr, rdt = _mat(R, "tri_inverse_x3")
        n = R.shape[0]
        if R.shape[1] != n:
            raise IFKFACBackendError("tri_inverse_x3: R must be square")
        Z = torch.empty((n, n), dtype=torch.float32, device=R.device)
        ws = self._ws(self.lib.ifk_tri_inverse_x3_workspace_size(n, rdt), R.device)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_tri_inverse_x3(self._stream(R.device), _ptr(R), rdt, ldr, n, _ptr(Z),
                                             n, _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_tri_inverse_x3")
        return Z

    def tri_inverse_bf16(self, R: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor,
                                                          torch.Tensor]:
        """tri_inverse in bf16 arithmetic, also returning the RNE bf16 copies
        (Z, Z^T) that precondition_apply_bf16 reads (their other triangle zero)."""
        R, ldr, rdt = _mat(R, "tri_inverse_bf16")
        n = R.shape[0]
        if R.shape[1] != n:
            raise IFKFACBackendError("tri_inverse_bf16: R must be square")
        Z = torch.empty((n, n), dtype=torch.float32, device=R.device)
        Zb = torch.empty((n, n), dtype=torch.bfloat16, device=R.device)
        ZT = torch.empty((n, n), dtype=torch.bfloat16, device=R.device)
        ws = self._ws(self.lib.ifk_tri_inverse_bf16_workspace_size(n), R.device)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_tri_inverse_bf16(self._stream(R.device), _ptr(R), rdt, ldr, n,
                                               _ptr(Z), n, _ptr(Zb), _ptr(ZT), n, _ptr(ws),
                                               ws.numel())
        _lib.check(rc, "ifk_tri_inverse_bf16")
        return Z, Zb, ZT

    def cond_estimate(self, R: torch.Tensor, Z: torch.Tensor) -> torch.Tensor:
        """kappa_2(R) estimate from R and its fp32 inverse Z, as a device float[1]
        (read it with the factor flags, after the stream has progressed)."""
        R, ldr, rdt = _mat(R, "cond_estimate")
        Zc, ldz, zdt = _mat(Z, "cond_estimate")
        n = R.shape[0]
        if R.shape != (n, n) or Zc.shape != (n, n) or zdt != IFK_F32:
            raise IFKFACBackendError("cond_estimate: R and Z must be n x n, Z fp32")
        out = torch.empty(1, dtype=torch.float32, device=R.device)
        ws = self._ws(self.lib.ifk_cond_estimate_workspace_size(n), R.device)
        with torch.cuda.device(R.device):
            rc = self.lib.ifk_cond_estimate(self._stream(R.device), _ptr(R), rdt, ldr, _ptr(Zc),
                                            ldz, n, _ptr(out), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_cond_estimate")
        return out

    def precondition_apply_bf16(self, grad: torch.Tensor, ZX2, ZG2) -> torch.Tensor:
        """precondition_apply in bf16 arithmetic from (Z_X, Z_X^T), (Z_G, Z_G^T)
        bf16 copies of tri_inverse_bf16 (views of them, e.g. trimmed, allowed)."""
        g, ldg, gdt = _mat(grad, "precondition_apply_bf16")
        if gdt != IFK_F32:
            g = g.float()
            ldg = g.stride(0)
        n_out, n_in = g.shape
        (ZXb, ZXt), (ZGb, ZGt) = ZX2, ZG2
        for name, t, n in (("Z_X", ZXb, n_in), ("Z_X^T", ZXt, n_in), ("Z_G", ZGb, n_out),
                           ("Z_G^T", ZGt, n_out)):
            _require_device(t, "precondition_apply_bf16")
            if t.dtype != torch.bfloat16 or t.shape != (n, n) or t.stride(1) != 1:
                raise IFKFACBackendError(f"precondition_apply_bf16: {name} must be an "
                                         f"{n} x {n} bf16 row-major matrix")
        if ZXb.stride(0) != ZXt.stride(0) or ZGb.stride(0) != ZGt.stride(0):
            raise IFKFACBackendError("precondition_apply_bf16: a side's two copies differ in "
                                     "row stride")
        nat = torch.empty((n_out, n_in), dtype=torch.float32, device=g.device)
        ws = self._ws(self.lib.ifk_precondition_apply_bf16_workspace_size(n_out, n_in), g.device)
        with torch.cuda.device(g.device):
            rc = self.lib.ifk_precondition_apply_bf16(
                self._stream(g.device), _ptr(g), n_out, n_in, ldg, _ptr(ZXb), _ptr(ZXt),
                ZXb.stride(0), _ptr(ZGb), _ptr(ZGt), ZGb.stride(0), _ptr(nat), n_in, _ptr(ws),
                ws.numel())
        _lib.check(rc, "ifk_precondition_apply_bf16")
        return nat

    def inverse_split_copies(self, Z: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        """bf16 halves of an fp32 inverse for precondition_apply_x3:
        (Z_hi, Z_lo, Z^T_hi, Z^T_lo), Z = Z_hi + Z_lo, each n x n row-major."""
        Zc, ldz, zdt = _mat(Z, "inverse_split_copies")
        n = Zc.shape[0]
        if Zc.shape != (n, n) or zdt != IFK_F32:
            raise IFKFACBackendError("inverse_split_copies: Z must be n x n fp32")
        out = torch.empty((4, n, n), dtype=torch.bfloat16, device=Zc.device)
        with torch.cuda.device(Zc.device):
            rc = self.lib.ifk_inverse_split_copies(self._stream(Zc.device), _ptr(Zc), ldz, n,
                                                   _ptr(out[0]), _ptr(out[1]), _ptr(out[2]),
                                                   _ptr(out[3]), n)
        _lib.check(rc, "ifk_inverse_split_copies")
        return tuple(out.unbind(0))

    def inverse_split_copies_batched(self, Zs) -> list:
        """inverse_split_copies for B inverses of one size, the halves of all of
        them in one (4, B, n, n) buffer: entry e gets the views
        (Z_hi, Z_lo, Z^T_hi, Z^T_lo) at a fixed stride from entry to entry, as
        precondition_apply_x3_batched takes them."""
        n = Zs[0].shape[0]
        dev = Zs[0].device
        out = torch.empty((4, len(Zs), n, n), dtype=torch.bfloat16, device=dev)
        for e, Z in enumerate(Zs):
            Zc, ldz, zdt = _mat(Z, "inverse_split_copies")
            if Zc.shape != (n, n) or zdt != IFK_F32:
                raise IFKFACBackendError("inverse_split_copies: Z must be n x n fp32")
            with torch.cuda.device(dev):
                rc = self.lib.ifk_inverse_split_copies(self._stream(dev), _ptr(Zc), ldz, n,
                                                       _ptr(out[0, e]), _ptr(out[1, e]),
                                                       _ptr(out[2, e]), _ptr(out[3, e]), n)
            _lib.check(rc, "ifk_inverse_split_copies")
        return [tuple(out[i, e] for i in range(4)) for e in range(len(Zs))]

    @staticmethod
    def entry_stride(ts) -> Optional[int]:
        """The element stride at which the same-shape tensors ts sit one after
        another in memory (one stride between every two consecutive ones, row
        stride and dtype alike), or None (len(ts) == 1: 0)."""
        if len(ts) == 1:
            return 0
        es = ts[0].element_size()
        d = ts[1].data_ptr() - ts[0].data_ptr()
        if d <= 0 or d % es:
            return None
        for a, b in zip(ts, ts[1:]):
            if (b.data_ptr() - a.data_ptr() != d or b.shape != a.shape or b.stride() != a.stride()
                    or b.dtype != a.dtype or b.device != a.device):
                return None
        return d // es

    def _batch_grads(self, grads, name):
        gs = []
        for g in grads:
            g, ldg, gdt = _mat(g, name)
            if gdt != IFK_F32:
                g = g.float()
                ldg = g.stride(0)
            gs.append((g, ldg))
        n_out, n_in = gs[0][0].shape
        ldg = gs[0][1]
        if any(g.shape != (n_out, n_in) or l != ldg or g.device != gs[0][0].device
               for g, l in gs):
            raise IFKFACBackendError(f"{name}: gradients differ in shape or row stride")
        ptrs = (ctypes.c_void_p * len(gs))(*[g.data_ptr() for g, _ in gs])
        return gs, ptrs, n_out, n_in, ldg

    def precondition_apply_bf16_batched(self, grads, ZX2s, ZG2s) -> torch.Tensor:
        """precondition_apply_bf16 for B layers of one shape in grouped launches
        (ifk_precondition_apply_bf16_batched): every layer's (Z_X, Z_X^T) and
        (Z_G, Z_G^T) copies at one fixed stride from layer to layer (views of
        one (B, n, n) buffer each, as the batched factor update returns them).
        Returns nat (B, n_out, n_in); entry e is bitwise the single-layer result."""
        name = "precondition_apply_bf16_batched"
        gs, ptrs, n_out, n_in, ldg = self._batch_grads(grads, name)
        B = len(gs)
        strides = []
        for side, n in ((ZX2s, n_in), (ZG2s, n_out)):
            for j in (0, 1):
                ts = [c[j] for c in side]
                for t in ts:
                    _require_device(t, name)
                    if t.dtype != torch.bfloat16 or t.shape != (n, n) or t.stride(1) != 1:
                        raise IFKFACBackendError(f"{name}: copies must be {n} x {n} bf16")
                st = self.entry_stride(ts)
                if st is None:
                    raise IFKFACBackendError(f"{name}: a side's copies are not at one stride")
                strides.append(st)
        if strides[0] != strides[1] or strides[2] != strides[3] or \
                ZX2s[0][0].stride(0) != ZX2s[0][1].stride(0) or \
                ZG2s[0][0].stride(0) != ZG2s[0][1].stride(0):
            raise IFKFACBackendError(f"{name}: a side's two copies differ in stride")
        dev = gs[0][0].device
        nat = torch.empty((B, n_out, n_in), dtype=torch.float32, device=dev)
        ws = self._ws(self.lib.ifk_precondition_apply_bf16_batched_workspace_size(B, n_out, n_in),
                      dev)
        (ZXb, ZXt), (ZGb, ZGt) = ZX2s[0], ZG2s[0]
        with torch.cuda.device(dev):
            rc = self.lib.ifk_precondition_apply_bf16_batched(
                self._stream(dev), B, ctypes.cast(ptrs, ctypes.c_void_p), n_out, n_in, ldg,
                _ptr(ZXb), _ptr(ZXt), ZXb.stride(0), strides[0], _ptr(ZGb), _ptr(ZGt),
                ZGb.stride(0), strides[2], _ptr(nat), n_in, n_out * n_in, _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_precondition_apply_bf16_batched")
        return nat

    def precondition_apply_x3_batched(self, grads, ZX4s, ZG4s) -> torch.Tensor:
        """precondition_apply_x3 for B layers of one shape in grouped launches
        (ifk_precondition_apply_x3_batched): each of the four halves of every
        side at one fixed stride from layer to layer (inverse_split_copies_batched
        makes them so).  Returns nat (B, n_out, n_in), bitwise the per-layer
        results."""
        name = "precondition_apply_x3_batched"
        gs, ptrs, n_out, n_in, ldg = self._batch_grads(grads, name)
        B = len(gs)
        sides = []
        for side, n in ((ZX4s, n_in), (ZG4s, n_out)):
            st = None
            for j in range(4):
                ts = [c[j] for c in side]
                for t in ts:
                    _require_device(t, name)
                    if t.dtype != torch.bfloat16 or t.shape != (n, n) or t.stride(1) != 1 or \
                            t.stride(0) != side[0][0].stride(0):
                        raise IFKFACBackendError(f"{name}: halves must be {n} x {n} bf16 with "
                                                 f"one row stride")
                sj = self.entry_stride(ts)
                if sj is None or (st is not None and sj != st):
                    raise IFKFACBackendError(f"{name}: a side's halves are not at one stride")
                st = sj
            sides.append(st)
        dev = gs[0][0].device
        nat = torch.empty((B, n_out, n_in), dtype=torch.float32, device=dev)
        ws = self._ws(self.lib.ifk_precondition_apply_x3_batched_workspace_size(B, n_out, n_in),
                      dev)
        with torch.cuda.device(dev):
            rc = self.lib.ifk_precondition_apply_x3_batched(
                self._stream(dev), B, ctypes.cast(ptrs, ctypes.c_void_p), n_out, n_in, ldg,
                *[_ptr(t) for t in ZX4s[0]], ZX4s[0][0].stride(0), sides[0],
                *[_ptr(t) for t in ZG4s[0]], ZG4s[0][0].stride(0), sides[1], _ptr(nat), n_in,
                n_out * n_in, _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_precondition_apply_x3_batched")
        return nat

    def precondition_apply_x3(self, grad: torch.Tensor, ZX4, ZG4) -> torch.Tensor:
        """precondition_apply at fp32 accuracy from the split copies of
        inverse_split_copies (views of them, e.g. trimmed, allowed)."""
        g, ldg, gdt = _mat(grad, "precondition_apply_x3")
        if gdt != IFK_F32:
            g = g.float()
            ldg = g.stride(0)
        n_out, n_in = g.shape
        for name, side, n in (("Z_X", ZX4, n_in), ("Z_G", ZG4, n_out)):
            if len(side) != 4:
                raise IFKFACBackendError(f"precondition_apply_x3: {name} needs four copies")
            for t in side:
                _require_device(t, "precondition_apply_x3")
                if t.dtype != torch.bfloat16 or t.shape != (n, n) or t.stride(1) != 1 or \
                        t.stride(0) != side[0].stride(0):
                    raise IFKFACBackendError(f"precondition_apply_x3: {name} copies must be "
                                             f"{n} x {n} bf16 row-major with one row stride")
        nat = torch.empty((n_out, n_in), dtype=torch.float32, device=g.device)
        ws = self._ws(self.lib.ifk_precondition_apply_x3_workspace_size(n_out, n_in), g.device)
        with torch.cuda.device(g.device):
            rc = self.lib.ifk_precondition_apply_x3(
                self._stream(g.device), _ptr(g), n_out, n_in, ldg, *[_ptr(t) for t in ZX4],
                ZX4[0].stride(0), *[_ptr(t) for t in ZG4], ZG4[0].stride(0), _ptr(nat), n_in,
                _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_precondition_apply_x3")
        return nat

    # -- Laplace consumer -------------------------------------------------------------
    def factor_evd(self, R: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(V, eig, sweeps): R^T R = V diag(eig) V^T from the upper triangle of R,
        eig descending (fp32); sweeps a device int32[1] (negative: not converged)."""
        Rc, ldr, rdt = _mat(R, "factor_evd")
        n = Rc.shape[0]
        if Rc.shape != (n, n):
            raise IFKFACBackendError("factor_evd: R must be square")
        V = torch.empty((n, n), dtype=torch.float32, device=Rc.device)
        eig = torch.empty(n, dtype=torch.float32, device=Rc.device)
        sweeps = torch.empty(1, dtype=torch.int32, device=Rc.device)
        ws = self._ws(self.lib.ifk_factor_evd_workspace_size(n), Rc.device)
        with torch.cuda.device(Rc.device):
            rc = self.lib.ifk_factor_evd(self._stream(Rc.device), _ptr(Rc), rdt, ldr, n, _ptr(V), n,
                                         _ptr(eig), _ptr(sweeps), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_factor_evd")
        return V, eig, sweeps

    def laplace_scales(self, d: torch.Tensor, sqrt_n: float, sqrt_lam: float) -> torch.Tensor:
        """1 / sqrt(sqrt_n d + sqrt_lam), fp32."""
        _require_device(d, "laplace_scales")
        dc = d.reshape(-1).float().contiguous()
        out = torch.empty_like(dc)
        with torch.cuda.device(dc.device):
            rc = self.lib.ifk_laplace_scales(self._stream(dc.device), _ptr(dc), dc.numel(),
                                             float(sqrt_n), float(sqrt_lam), _ptr(out))
        _lib.check(rc, "ifk_laplace_scales")
        return out

    def laplace_sample_(self, W_map: torch.Tensor, W: torch.Tensor, U_G: torch.Tensor,
                        s_G: torch.Tensor, U_A: torch.Tensor, s_A: torch.Tensor,
                        Xi: torch.Tensor) -> None:
        """W (fp32 n_out x n_in, row-major, in place) = W_map + U_G diag(s_G) Xi
        diag(s_A) U_A^T."""
        n_out, n_in = Xi.shape
        mats = {}
        for name, t, shape in (("W_map", W_map, (n_out, n_in)), ("W", W, (n_out, n_in)),
                               ("U_G", U_G, (n_out, n_out)), ("U_A", U_A, (n_in, n_in)),
                               ("Xi", Xi, (n_out, n_in))):
            _require_device(t, "laplace_sample")
            if t.dtype != torch.float32 or t.shape != shape or t.stride(1) != 1:
                raise IFKFACBackendError(f"laplace_sample: {name} must be fp32 {shape} row-major")
            mats[name] = t
        for name, t, n in (("s_G", s_G, n_out), ("s_A", s_A, n_in)):
            if t.dtype != torch.float32 or t.numel() != n or not t.is_contiguous():
                raise IFKFACBackendError(f"laplace_sample: {name} must be fp32 of length {n}")
        ws = self._ws(self.lib.ifk_laplace_sample_workspace_size(n_out, n_in), W.device)
        with torch.cuda.device(W.device):
            rc = self.lib.ifk_laplace_sample(
                self._stream(W.device), _ptr(W_map), W_map.stride(0), _ptr(W), W.stride(0), n_out,
                n_in, _ptr(U_G), U_G.stride(0), _ptr(s_G), _ptr(U_A), U_A.stride(0), _ptr(s_A),
                _ptr(Xi), Xi.stride(0), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_laplace_sample")

    # -- Classic K-FAC control ------------------------------------------------------
    def gram_accumulate_(self, S: torch.Tensor, X: torch.Tensor, beta: float) -> None:
        """S = beta S + X^T X in place (S fp32 n x n contiguous, X p x n)."""
        Xc, ldx, xdt = _mat(X, "gram_accumulate")
        p, n = Xc.shape
        _require_device(S, "gram_accumulate")
        if S.dtype != torch.float32 or S.shape != (n, n) or S.stride(1) != 1:
            raise IFKFACBackendError("gram_accumulate: S must be an n x n fp32 row-major matrix")
        ws = self._ws(self.lib.ifk_gram_accumulate_workspace_size(n), Xc.device)
        with torch.cuda.device(Xc.device):
            rc = self.lib.ifk_gram_accumulate(self._stream(Xc.device), _ptr(Xc), xdt, p, n, ldx,
                                              _ptr(S), S.stride(0), float(beta), _ptr(ws),
                                              ws.numel())
        _lib.check(rc, "ifk_gram_accumulate")

    def axpby(self, alpha: float, X: torch.Tensor, beta: float,
              Y: Optional[torch.Tensor] = None) -> torch.Tensor:
        """alpha X + beta Y (fp32; a new tensor when Y is None, else Y in place)."""
        Xc, ldx, xdt = _mat(X, "axpby")
        if xdt != IFK_F32:
            raise IFKFACBackendError("axpby: X must be fp32")
        rows, cols = Xc.shape
        if Y is None:
            Y = torch.empty((rows, cols), dtype=torch.float32, device=Xc.device)
            beta = 0.0
        elif Y.dtype != torch.float32 or Y.shape != Xc.shape or Y.stride(1) != 1:
            raise IFKFACBackendError("axpby: Y must match X (fp32, row-major)")
        with torch.cuda.device(Xc.device):
            rc = self.lib.ifk_axpby(self._stream(Xc.device), float(alpha), _ptr(Xc), ldx,
                                    float(beta), _ptr(Y), Y.stride(0), rows, cols)
        _lib.check(rc, "ifk_axpby")
        return Y

    def inv_spd_damped(self, A: torch.Tensor, damping: float) -> torch.Tensor:
        """(A + damping I)^{-1} in fp32 (Cholesky and triangular inverse)."""
        Ac, lda, adt = _mat(A, "inv_spd_damped")
        n = Ac.shape[0]
        if Ac.shape != (n, n):
            raise IFKFACBackendError("inv_spd_damped: A must be square")
        X = torch.empty((n, n), dtype=torch.float32, device=Ac.device)
        ws = self._ws(self.lib.ifk_inv_spd_damped_workspace_size(n), Ac.device)
        with torch.cuda.device(Ac.device):
            rc = self.lib.ifk_inv_spd_damped(self._stream(Ac.device), _ptr(Ac), adt, n, lda,
                                             float(damping), _ptr(X), n, _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_inv_spd_damped")
        return X

    def classic_precondition(self, grad: torch.Tensor, A_inv: torch.Tensor,
                             G_inv: torch.Tensor) -> torch.Tensor:
        """G_inv grad A_inv in fp32."""
        g, ldg, gdt = _mat(grad, "classic_precondition")
        if gdt != IFK_F32:
            g = g.float()
            ldg = g.stride(0)
        n_out, n_in = g.shape
        Ai, ldai, adt = _mat(A_inv, "classic_precondition")
        Gi, ldgi, gidt = _mat(G_inv, "classic_precondition")
        if adt != IFK_F32 or gidt != IFK_F32 or Ai.shape != (n_in, n_in) or \
                Gi.shape != (n_out, n_out):
            raise IFKFACBackendError("classic_precondition: inverses must be fp32 and match grad")
        nat = torch.empty((n_out, n_in), dtype=torch.float32, device=g.device)
        ws = self._ws(self.lib.ifk_classic_precondition_workspace_size(n_out, n_in), g.device)
        with torch.cuda.device(g.device):
            rc = self.lib.ifk_classic_precondition(self._stream(g.device), _ptr(g), n_out, n_in,
                                                   ldg, _ptr(Ai), ldai, _ptr(Gi), ldgi, _ptr(nat),
                                                   n_in, _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_classic_precondition")
        return nat

    def precondition(self, grad: torch.Tensor, R_X: torch.Tensor, R_G: torch.Tensor,
                     math: int) -> torch.Tensor:
        g, ldg, gdt = _mat(grad, "precondition")
        if gdt != IFK_F32:
            g = g.float()
            ldg = g.stride(0)
        RX, ldrx, xdt = _mat(R_X, "precondition")
        RG, ldrg, gdt2 = _mat(R_G, "precondition")
        if xdt != gdt2:
            RX = RX.float()
            RG = RG.float()
            ldrx, ldrg, xdt = RX.stride(0), RG.stride(0), IFK_F32
        n_out, n_in = g.shape
        if RX.shape != (n_in, n_in) or RG.shape != (n_out, n_out):
            raise IFKFACBackendError(
                f"precondition: shapes grad {tuple(g.shape)}, R_X {tuple(RX.shape)}, "
                f"R_G {tuple(RG.shape)} do not match")
        nat = torch.empty((n_out, n_in), dtype=torch.float32, device=g.device)
        ws = self._ws(self.lib.ifk_precondition_workspace_size(n_out, n_in, int(math)), g.device)
        with torch.cuda.device(g.device):
            rc = self.lib.ifk_precondition(self._stream(g.device), _ptr(g), n_out, n_in, ldg,
                                           _ptr(RX), ldrx, _ptr(RG), ldrg, xdt, _ptr(nat), n_in,
                                           int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_precondition")
        return nat

    def precondition_apply(self, grad: torch.Tensor, Z_X: torch.Tensor, Z_G: torch.Tensor,
                           math: int) -> torch.Tensor:
        g, ldg, gdt = _mat(grad, "precondition_apply")
        if gdt != IFK_F32:
            g = g.float()
            ldg = g.stride(0)
        n_out, n_in = g.shape
        ZX, ldzx, _ = _mat(Z_X, "precondition_apply")
        ZG, ldzg, _ = _mat(Z_G, "precondition_apply")
        if ZX.dtype != torch.float32 or ZG.dtype != torch.float32:
            raise IFKFACBackendError("precondition_apply: inverses must be fp32")
        if ZX.shape != (n_in, n_in) or ZG.shape != (n_out, n_out):
            raise IFKFACBackendError("precondition_apply: shape mismatch")
        nat = torch.empty((n_out, n_in), dtype=torch.float32, device=g.device)
        ws = self._ws(self.lib.ifk_precondition_apply_workspace_size(n_out, n_in, int(math)),
                      g.device)
        with torch.cuda.device(g.device):
            rc = self.lib.ifk_precondition_apply(self._stream(g.device), _ptr(g), n_out, n_in, ldg,
                                                 _ptr(ZX), ldzx, _ptr(ZG), ldzg, _ptr(nat), n_in,
                                                 int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_precondition_apply")
        return nat

    def precondition_bias(self, g: torch.Tensor, Z_G: torch.Tensor) -> torch.Tensor:
        _require_device(g, "precondition_bias")
        gv = g.reshape(-1)
        if gv.dtype != torch.float32:
            gv = gv.float()
        gv = gv.contiguous()
        n_out = gv.numel()
        ZG, ldzg, _ = _mat(Z_G, "precondition_bias")
        if ZG.shape != (n_out, n_out) or ZG.dtype != torch.float32:
            raise IFKFACBackendError("precondition_bias: shape/dtype mismatch")
        out = torch.empty(n_out, dtype=torch.float32, device=gv.device)
        ws = self._ws(self.lib.ifk_precondition_bias_workspace_size(n_out), gv.device)
        with torch.cuda.device(gv.device):
            rc = self.lib.ifk_precondition_bias(self._stream(gv.device), _ptr(gv), n_out, _ptr(ZG),
                                                ldzg, _ptr(out), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_precondition_bias")
        return out

    def release_stream_state(self, device, stream=None) -> None:
        """Free the helper streams and events the library keeps for (device,
        stream) -- the current stream by default (ifk_release_stream_state)."""
        dev = torch.device(device)
        with torch.cuda.device(dev):
            st = stream if stream is not None else torch.cuda.current_stream(dev)
            rc = self.lib.ifk_release_stream_state(ctypes.c_void_p(st.cuda_stream))
        _lib.check(rc, "ifk_release_stream_state")

    def momentum_update_(self, nat: torch.Tensor, buf: Optional[torch.Tensor], W: torch.Tensor,
                         lr: float, momentum: float, weight_decay: float, buf_init: bool) -> None:
        _require_device(W, "momentum_update")
        if W.dtype != torch.float32 or not W.is_contiguous():
            raise IFKFACBackendError("momentum_update: W must be contiguous fp32")
        natc = nat.reshape(W.shape)
        if natc.dtype != torch.float32:
            natc = natc.float()
        natc = natc.contiguous()
        if buf is not None and (buf.dtype != torch.float32 or not buf.is_contiguous()
                                or buf.numel() != W.numel()):
            raise IFKFACBackendError("momentum_update: buf must match W")
        with torch.cuda.device(W.device):
            rc = self.lib.ifk_momentum_update(self._stream(W.device), _ptr(natc), _ptr(buf),
                                              _ptr(W), W.numel(), float(lr), float(momentum),
                                              float(weight_decay), 1 if buf_init else 0)
        _lib.check(rc, "ifk_momentum_update")

    # -- bf16_linalg counterparts --------------------------------------------------
    def geqrf_r(self, A: torch.Tensor, out_dtype: torch.dtype, math: int) -> torch.Tensor:
        A, lda, adt = _mat(A, "geqrf_r")
        m, n = A.shape
        R = torch.empty((n, n), dtype=out_dtype, device=A.device)
        ws = self._ws(self.lib.ifk_geqrf_r_workspace_size(m, n), A.device)
        with torch.cuda.device(A.device):
            rc = self.lib.ifk_geqrf_r(self._stream(A.device), _ptr(A), adt, m, n, lda, _ptr(R),
                                      _DT[out_dtype], n, int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_geqrf_r")
        return R

    def trsm(self, R: torch.Tensor, B: torch.Tensor, upper: bool, out_dtype: torch.dtype,
             math: int) -> torch.Tensor:
        R, ldr, rdt = _mat(R, "trsm")
        B, ldb, bdt = _mat(B, "trsm")
        n, k = B.shape
        X = torch.empty((n, k), dtype=out_dtype, device=B.device)
        ws = self._ws(self.lib.ifk_trsm_workspace_size(n, k), B.device)
        with torch.cuda.device(B.device):
            rc = self.lib.ifk_trsm(self._stream(B.device), _ptr(R), rdt, n, ldr, 1 if upper else 0,
                                   _ptr(B), bdt, k, ldb, _ptr(X), _DT[out_dtype], max(k, 1),
                                   int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_trsm")
        return X

    def potrf(self, A: torch.Tensor, out_dtype: torch.dtype, math: int) -> torch.Tensor:
        A, lda, adt = _mat(A, "potrf")
        n = A.shape[0]
        L = torch.empty((n, n), dtype=out_dtype, device=A.device)
        ws = self._ws(self.lib.ifk_potrf_workspace_size(n), A.device)
        with torch.cuda.device(A.device):
            rc = self.lib.ifk_potrf(self._stream(A.device), _ptr(A), adt, n, lda, _ptr(L),
                                    _DT[out_dtype], n, int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_potrf")
        return L

    def inv_spd(self, A: torch.Tensor, out_dtype: torch.dtype, math: int) -> torch.Tensor:
        A, lda, adt = _mat(A, "inv_spd")
        n = A.shape[0]
        X = torch.empty((n, n), dtype=out_dtype, device=A.device)
        ws = self._ws(self.lib.ifk_inv_spd_workspace_size(n), A.device)
        with torch.cuda.device(A.device):
            rc = self.lib.ifk_inv_spd(self._stream(A.device), _ptr(A), adt, n, lda, _ptr(X),
                                      _DT[out_dtype], n, int(math), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_inv_spd")
        return X

    def gemm(self, A: torch.Tensor, B: torch.Tensor, trans_a: bool = False,
             trans_b: bool = False, math: int = MATH_F32, alpha: float = 1.0,
             beta: float = 0.0, C: Optional[torch.Tensor] = None, tri_a: int = 0,
             tri_b: int = 0) -> torch.Tensor:
        """C = alpha op(A) op(B) + beta C; tri_x = 1 / 2 declares op(X) upper /
        lower triangular (its other triangle is not read)."""
        A, lda, adt = _mat(A, "gemm")
        B, ldb, bdt = _mat(B, "gemm")
        m = A.shape[1] if trans_a else A.shape[0]
        k = A.shape[0] if trans_a else A.shape[1]
        kb = B.shape[1] if trans_b else B.shape[0]
        n = B.shape[0] if trans_b else B.shape[1]
        if k != kb:
            raise IFKFACBackendError("gemm: inner dimensions differ")
        if C is None:
            C = torch.zeros((m, n), dtype=torch.float32, device=A.device)
        ws = self._ws(self.lib.ifk_gemm_workspace_size(m, n), A.device)
        with torch.cuda.device(A.device):
            rc = self.lib.ifk_gemm(self._stream(A.device), int(math), m, n, k, float(alpha),
                                   _ptr(A), adt, lda, int(trans_a) | (int(tri_a) << 1),
                                   _ptr(B), bdt, ldb, int(trans_b) | (int(tri_b) << 1),
                                   float(beta), _ptr(C), C.stride(0), _ptr(ws), ws.numel())
        _lib.check(rc, "ifk_gemm")
        return C


_BACKEND = None


def get_backend():
    """The active backend; loads the HIP library on first use."""
    global _BACKEND
    if _BACKEND is None:
        _BACKEND = HipBackend()
    return _BACKEND


def set_backend(backend):
    """Install another backend object (test doubles); returns the previous one."""
    global _BACKEND
    prev = _BACKEND
    _BACKEND = backend
    return prev


_SIDE_STREAMS = {}


def _side_streams(device: torch.device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _SIDE_STREAMS:
        with torch.cuda.device(idx):
            _SIDE_STREAMS[idx] = (torch.cuda.Stream(), torch.cuda.Stream())  # default priority
    return _SIDE_STREAMS[idx]


def _tensors(obj):
    if isinstance(obj, torch.Tensor):
        yield obj
    elif isinstance(obj, (tuple, list)):
        for o in obj:
            yield from _tensors(o)


def run_pair(device: torch.device, fa, fb, b_first: bool = False):
    """Run fa() and fb() concurrently on two side streams of `device`, after the
    current stream's pending work; the current stream then waits for both.
    Used for the independent input-side and output-side factor work (fold +
    finalize, triangular inverse).  b_first enqueues fb() before fa() (the
    longer call first, so its GPU work starts while the host enqueues the
    other).  The call enqueued first always runs on the same side stream,
    whichever of fa and fb it is: the library keeps its helper streams per
    calling stream, and a layer's longer factorisation ran about 3 ms slower
    per step (Linear 11008 -> 4096, p = 16384: 15.4 against 12.5 ms) on the
    side stream whose helpers had carried the shorter side of another layer
    (4096 -> 11008) than on the one whose helpers had carried the longer.
    On a CPU device the two calls simply run in order."""
    if device.type != "cuda":
        return fa(), fb()
    main = torch.cuda.current_stream(device)
    s1, s2 = _side_streams(device)
    s1.wait_stream(main)
    s2.wait_stream(main)
    if b_first:
        with torch.cuda.stream(s2):
            rb = fb()
        with torch.cuda.stream(s1):
            ra = fa()
    else:
        with torch.cuda.stream(s2):
            ra = fa()
        with torch.cuda.stream(s1):
            rb = fb()
    main.wait_stream(s1)
    main.wait_stream(s2)
    for t in list(_tensors(ra)) + list(_tensors(rb)):
        if t.is_cuda:
            t.record_stream(main)
    return ra, rb


def inv_sqrt(rows: int) -> float:
    return 1.0 / _math.sqrt(rows)
