"""Forward/backward hooks that keep each layer's streaming R factors.

Counterpart of ``RawActivationHooks`` (ifkfac/activation_hooks.py:87-653): the
same constructor, modes (streaming, ``batched``, ``deferred``), row
subsampling, Conv2d im2col, bias augmentation, skip rules and public methods.
The numerical work goes to the HIP fold kernel: each tracked layer owns two
persistent ``n x n`` fp32 buffers (input side X, output-gradient side G) that
the fold updates in place, and ``_R_X[module]`` / ``_R_G[module]`` are views
of the valid rows, shaped ``(min(rows, n), n)`` exactly as the reference's
running factors are.
"""
from __future__ import annotations

import collections
import logging
import math
import warnings
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from ._backend import MATH_BF16, MATH_F32, get_backend, run_pair
from .gram_estimator import GramMatrixEstimator

logger = logging.getLogger(__name__)

warnings.filterwarnings("ignore", message="Full backward hook is firing", category=UserWarning)

# Pivot threshold of the Gram-route streaming fold (bf16 arithmetic): a fold
# whose Cholesky meets a pivot below this fraction of its column's Gram
# diagonal is redone by the panel fold.  At 1e-4 the Gram route's rounding
# (about 2^-17 of the diagonal per product) stays under 8% of any pivot it
# keeps, and its factor's backward error (R^T R against the Gram matrix of
# the bf16-rounded rows) stays far below the bf16 panel fold's.
GRAM_FOLD_TOL = 1e-4
# A fold the Gram route refuses (its pivot test found the rows ill-conditioned
# or rank-deficient) is redone by the panel fold in fp32 arithmetic: on such
# rows the bf16 panel fold drifts along a stream (the output-gradient side of
# a ViT-B qkv projection, columns 768.. zero: 6.3e-2 relative Gram error after
# 120 folds of 4096 rows, against 7e-5 in fp32 arithmetic), while the
# reference keeps its running factor in fp32 (triangular.py:246-307).
REFUSED_FOLD_MATH = MATH_F32


class FoldStatusQueue:
    """Gram-route folds whose status is read without blocking the host.

    A fold by the Gram route either writes the factor of [R; X] (status 1) or
    leaves R as it was (status 2: a pivot below GRAM_FOLD_TOL of its Gram
    diagonal).  Instead of reading the status at once -- a blocking device
    read inside a forward or backward hook, which the reference's hooks never
    make (activation_hooks.py:579-580, 642-643) -- ``push`` copies it to
    pinned host memory behind the fold on the same stream, records an event,
    and keeps a copy of the chunk (the caller's tensor may be changed in
    place once the hook returns -- autograd reuses gradient buffers -- while a
    refused chunk is read again later).  ``poll`` resolves, without blocking,
    the folds whose
    event has completed: a refused chunk is then folded by the panel path
    into the running factor as it is at that point (R^T R is the sum of the
    folded chunks' Gram matrices, so the order of the folds does not change
    the factor).  ``drain`` resolves the rest, blocking; readers of the
    factors call it first.  At most ``cap`` folds wait (the kept chunks hold
    memory); beyond that the oldest is resolved blocking.  The pinned status
    words and their events come from one process-wide pool (a pinned
    allocation costs far more than a fold's launches)."""

    # (pinned int32[1], event) pairs per device, shared by all queues
    _pool: Dict[int, List[tuple]] = {}

    def __init__(self, cap: int = 32):
        self.cap = cap
        self._q: collections.deque = collections.deque()
        self.refused = 0               # refused folds resolved so far

    def __len__(self) -> int:
        return len(self._q)

    def push(self, st: torch.Tensor, buf: torch.Tensor, chunk: torch.Tensor,
             math_: int, owned: bool = False) -> None:
        """Queue the fold of ``chunk`` into ``buf`` whose status is ``st``;
        ``owned``: the chunk is a private copy no one changes (kept as is)."""
        if st.device.type != "cuda":
            # a host backend: the status is on the host already
            self._resolve(int(st.reshape(-1)[0].item()), buf, chunk, math_)
            return
        if len(self._q) >= self.cap:
            self._pop(block=True)
        free = FoldStatusQueue._pool.setdefault(st.device.index, [])
        if not free:
            with torch.cuda.device(st.device):
                block = torch.empty(64, dtype=torch.int32, pin_memory=True)
                free.extend((block[i:i + 1], torch.cuda.Event()) for i in range(64))
        slot, ev = free.pop()
        if not owned:
            chunk = chunk.clone()   # on the stream, behind the fold that read it
        be = get_backend()
        if hasattr(be, "status_to_host"):
            # a kernel store: a copy-engine transfer between two folds' kernels
            # would stall the stream for far longer than the folds take
            be.status_to_host(st.reshape(-1)[:1], slot)
        else:
            slot.copy_(st.reshape(-1)[:1], non_blocking=True)
        ev.record()
        self._q.append((slot, ev, st.device.index, buf, chunk, math_))

    def poll(self) -> None:
        while self._q and self._q[0][1].query():
            self._pop(block=False)

    def drain(self) -> None:
        while self._q:
            self._pop(block=True)

    def discard(self) -> None:
        """Forget the waiting folds (their factors are being dropped)."""
        while self._q:
            slot, ev, dev, _, _, _ = self._q.popleft()
            ev.synchronize()     # the slot is reused only once its copy is done
            FoldStatusQueue._pool[dev].append((slot, ev))

    def _pop(self, block: bool) -> None:
        slot, ev, dev, buf, chunk, math_ = self._q.popleft()
        if block:
            ev.synchronize()
        st = int(slot[0])
        FoldStatusQueue._pool[dev].append((slot, ev))
        self._resolve(st, buf, chunk, math_)

    def _resolve(self, st: int, buf: torch.Tensor, chunk: torch.Tensor, math_: int) -> None:
        if st == 1:
            return
        self.refused += 1
        n = buf.shape[1]
        logger.debug("fold of %d rows into a %d-column factor: Gram route refused, panel fold",
                     chunk.shape[0], n)
        get_backend().fold_(buf, n, chunk, REFUSED_FOLD_MATH)


def fold_chunk(buf: torch.Tensor, r_in: int, chunk: torch.Tensor, math_: int,
               queue: Optional[FoldStatusQueue] = None, owned: bool = False) -> int:
    """Fold ``chunk`` into ``buf`` (n x n fp32, rows [0, r_in) valid); returns
    the new row count.  In bf16 arithmetic a fold whose result is square goes by
    the Gram matrix and the blocked Cholesky (about 3x faster than the panel
    fold), and a fold the Gram route refuses leaves buf as it was for the
    panel fold (in fp32 arithmetic: REFUSED_FOLD_MATH).  Without ``queue`` the
    status is read at once (the host waits for that fold).  With it the
    status is read later (FoldStatusQueue), so
    the next folds run before a refusal is known: the Gram route is then
    taken where the folded rows stay well spread whatever happens -- into a
    square running factor (r_in = n), or with at least 2n rows in all -- and
    rows [r_in, n) are zeroed first, so that a refused fold leaves an n-row
    factor whose extra rows contribute nothing.  A nearly square first fold
    (n <= r_in + p < 2n: its Gram matrix is often too ill-conditioned, and a
    refusal would leave the following folds a rank-deficient factor, which
    they would refuse in turn) takes the panel fold directly.  ``owned``: the
    chunk is a private copy (the queue keeps it without copying)."""
    be = get_backend()
    n = buf.shape[1]
    p = chunk.shape[0]
    if math_ == MATH_BF16 and r_in + p >= n:
        if queue is not None:
            if r_in < n and r_in + p < 2 * n:
                return be.fold_(buf, r_in, chunk, math_)
            if r_in < n:
                buf[r_in:].zero_()
            queue.push(be.fold_gram_(buf, r_in, chunk, GRAM_FOLD_TOL), buf, chunk, math_, owned)
            return n
        if int(be.fold_gram_(buf, r_in, chunk, GRAM_FOLD_TOL).item()) == 1:
            return n
        logger.debug("fold of %d rows into a %d-column factor: Gram route refused, panel fold",
                     chunk.shape[0], n)
        return be.fold_(buf, r_in, chunk, REFUSED_FOLD_MATH)
    return be.fold_(buf, r_in, chunk, math_)


class RowAccumulator:
    """Small chunks of one running factor, held until one fold of them pays.

    A fold's cost at a given width is mostly its chain of latency-bound
    launches, whatever the rows; and a fold whose result is not a square
    factor, or barely one, cannot take the Gram route.  In bf16 arithmetic a
    chunk that would make such a fold -- fewer than 2n rows in all into a
    partial factor, or fewer than 2n into a square one (n once the copies
    held reach HOLD_BYTES) -- is kept (a copy) and folded with the chunks
    after it once they reach that many rows.  RᵀR is the sum of the folded
    rows' Gram matrices, so the factor does not depend on how the rows are
    grouped.  fp32 arithmetic folds every chunk as it comes.  Readers of the
    factor drain the rows held.  ``add`` folds the rows once due; ``offer``
    hands them to a caller that folds them with other factors' (FoldGroups).

    Measured (one ViT-B block's capture, 4096-row batches, widths 768 to
    3072): folds into a square factor at n rows 3.65 ms per batch, at 2n rows
    2.37 (the 2304- and 3072-wide factors' chains run every other batch)."""

    # rows of a fold into a square factor, in widths, while the copies held
    # stay below HOLD_BYTES; past that, a width's worth of rows is due
    SQUARE_ROWS = 2
    HOLD_BYTES = 256 << 20

    def __init__(self) -> None:
        self.chunks: List[torch.Tensor] = []
        self.rows = 0
        self.nbytes = 0

    def _due(self, r_in: int, n: int, rows: int, nbytes: int) -> bool:
        if r_in < n:
            return r_in + rows >= 2 * n
        return rows >= self.SQUARE_ROWS * n or (rows >= n and nbytes >= self.HOLD_BYTES)

    @staticmethod
    def _bytes(chunk: torch.Tensor) -> int:
        return chunk.numel() * chunk.element_size()

    def add(self, buf: torch.Tensor, r_in: int, chunk: torch.Tensor, math_: int,
            queue: Optional["FoldStatusQueue"] = None) -> int:
        n = buf.shape[1]
        if not self.chunks and (math_ != MATH_BF16 or
                                self._due(r_in, n, chunk.shape[0], self._bytes(chunk))):
            return fold_chunk(buf, r_in, chunk, math_, queue)
        self.chunks.append(chunk.detach().clone(memory_format=torch.contiguous_format))
        self.rows += chunk.shape[0]
        self.nbytes += self._bytes(chunk)
        if self._due(r_in, n, self.rows, self.nbytes):
            return self.drain(buf, r_in, math_, queue)
        return r_in

    def offer(self, r_in: int, n: int, chunk: torch.Tensor,
              owned: bool = False) -> Tuple[Optional[torch.Tensor], bool]:
        """Hold ``chunk`` (a copy unless ``owned``) unless the rows held with it
        make a fold that pays; then return them as one chunk, forgetting them:
        (rows, whether they are a private copy), or (None, False) while held.
        For a caller that folds them itself (a grouped fold)."""
        if not self.chunks and self._due(r_in, n, chunk.shape[0], self._bytes(chunk)):
            return chunk, owned
        self.chunks.append(chunk if owned else
                           chunk.detach().clone(memory_format=torch.contiguous_format))
        self.rows += chunk.shape[0]
        self.nbytes += self._bytes(chunk)
        if self._due(r_in, n, self.rows, self.nbytes):
            return self.take(), True
        return None, False

    def take(self) -> Optional[torch.Tensor]:
        """The rows held, as one chunk (None if none), and forget them."""
        if not self.chunks:
            return None
        X = self.chunks[0] if len(self.chunks) == 1 else torch.cat(self.chunks, dim=0)
        self.chunks, self.rows, self.nbytes = [], 0, 0
        return X

    def drain(self, buf: torch.Tensor, r_in: int, math_: int,
              queue: Optional["FoldStatusQueue"] = None) -> int:
        X = self.take()
        return r_in if X is None else fold_chunk(buf, r_in, X, math_, queue)


class FoldGroups:
    """Gram-route folds of several running factors, held for one batched fold
    per shape.

    In bf16 arithmetic a fold by the Gram route costs mostly its chain of
    latency-bound launches, and the batched Gram-route fold
    (``fold_gram_batched_``) takes any number of same-shape folds through one
    chain, each factor bit for bit what its own fold gives.  The hooks get a
    model's chunks one layer at a time; ``hold`` keeps a copy of a chunk with
    its factor's buffer and row count, and ``flush`` folds everything held: one
    batched fold per (rows, columns, dtype, rows in the factor) group, the
    statuses read later (FoldStatusQueue).  A factor holds at most one chunk:
    its owner flushes before a second one and before anything reads or changes
    the factor.  A ViT-B-shaped model of 12 blocks (96 factors, 4096-row
    chunks): 83.6 -> 29.7 ms per batch."""

    # held copies beyond this many bytes are folded at once
    HOLD_BYTES = 4 << 30

    def __init__(self) -> None:
        self._items: Dict[tuple, tuple] = {}   # key -> (buf, r_in, chunk)
        self._bytes = 0

    def __contains__(self, key) -> bool:
        return key in self._items

    def __len__(self) -> int:
        return len(self._items)

    def hold(self, key, buf: torch.Tensor, r_in: int, chunk: torch.Tensor,
             owned: bool = False) -> bool:
        """Keep ``chunk`` for ``buf``'s next fold (a due one); True when the
        held copies have reached HOLD_BYTES and should be folded now."""
        if key in self._items:
            raise RuntimeError("FoldGroups.hold: the factor already holds a chunk")
        X = chunk if owned else chunk.detach().clone(memory_format=torch.contiguous_format)
        self._items[key] = (buf, r_in, X)
        self._bytes += X.numel() * X.element_size()
        return self._bytes >= self.HOLD_BYTES

    def discard(self) -> None:
        self._items.clear()
        self._bytes = 0

    # A square group of width n joins a wider square group of width N (same
    # rows per chunk) when n >= MERGE_RATIO * N: its entries ride the wider
    # group's chain of launches, embedded as [[R, 0], [0, I]] with the chunk
    # padded by zero columns, whose factor is [[R', 0], [0, I]] with R' the
    # entry's own.  That costs the entry (N / n)^2 of its Gram flops and saves
    # its own chain (a ViT-B block's 2304-wide side with its two 3072-wide
    # ones).
    MERGE_RATIO = 0.7

    def flush(self, math_: int, queue: FoldStatusQueue) -> None:
        items = list(self._items.values())
        self.discard()
        if not items:
            return
        be = get_backend()
        groups: Dict[tuple, list] = {}
        for buf, r_in, X in items:
            groups.setdefault((tuple(X.shape), X.dtype, X.device, r_in), []).append((buf, X))
        batched = hasattr(be, "fold_gram_batched_")
        # narrower square groups into the widest square group of their rows
        pads: Dict[tuple, list] = {}
        if batched:
            square = [k for k in groups if k[3] == k[0][1]]
            for k in sorted(square, key=lambda k: k[0][1]):
                if k in pads:   # it takes narrower ones itself
                    continue
                p, n = k[0]
                wide = [w for w in square if w[0][0] == p and w[1:3] == k[1:3] and
                        w[0][1] > n and n >= self.MERGE_RATIO * w[0][1] and w in groups]
                if wide:
                    w = max(wide, key=lambda w: w[0][1])
                    pads.setdefault(w, []).extend(groups.pop(k))
        for key, ent in groups.items():
            shape, r_in = key[0], key[3]
            n = shape[1]
            extra = pads.get(key, [])
            if len(ent) + len(extra) == 1 or not batched:
                for buf, X in ent:
                    fold_chunk(buf, r_in, X, math_, queue, owned=True)
                continue
            bufs = [b for b, _ in ent]
            chunks = [X for _, X in ent]
            if r_in < n:
                # as fold_chunk: a refused fold then leaves n rows whose extra
                # rows contribute nothing
                for b in bufs:
                    b[r_in:].zero_()
            embedded = []
            for buf, X in extra:
                m = buf.shape[0]
                P = torch.zeros((n, n), dtype=torch.float32, device=buf.device)
                P[:m, :m].copy_(buf)
                d = torch.arange(m, n, device=buf.device)
                P[d, d] = 1.0
                Xp = torch.zeros((X.shape[0], n), dtype=X.dtype, device=X.device)
                Xp[:, :m].copy_(X)
                bufs.append(P)
                chunks.append(Xp)
                embedded.append((buf, X, P, m))
            st = be.fold_gram_batched_(bufs, r_in, chunks, GRAM_FOLD_TOL)
            for e, (buf, X) in enumerate(ent):
                queue.push(st[e:e + 1], buf, X, math_, owned=True)
            for e, (buf, X, P, m) in enumerate(embedded, start=len(ent)):
                # a refused entry's P is as it was: the copy back changes nothing
                buf.copy_(P[:m, :m])
                queue.push(st[e:e + 1], buf, X, math_, owned=True)


def grouped_gram_finalize(items, damping: float, out_dtype: torch.dtype,
                          merge_ratio: float = FoldGroups.MERGE_RATIO) -> dict:
    """The damped factors of square running factors by the Gram route, one
    batched call per (width, rows folded, device) group instead of one call
    each; a narrower group rides a wider one (same rows, width n >=
    merge_ratio * N) embedded as [[R, 0], [0, I]], whose damped factor has
    the entry's own in its leading n x n block.  items: (key, R (n x n fp32),
    rows).  Returns key -> (R_damped, status int32[1], kappa bound float32[1])
    with the status of ``fold_finalize`` (2: redo by the panel path)."""
    be = get_backend()
    groups: Dict[tuple, list] = {}
    for key, R, rows in items:
        groups.setdefault((R.shape[1], rows, R.device), []).append((key, R))
    pads: Dict[tuple, list] = {}
    for k in sorted(groups, key=lambda k: k[0]):
        if k in pads:
            continue
        n = k[0]
        wide = [w for w in groups if w[1:] == k[1:] and w[0] > n and n >= merge_ratio * w[0]
                and w is not k]
        if wide:
            w = max(wide, key=lambda w: w[0])
            pads.setdefault(w, []).extend(groups.pop(k))
    out: dict = {}
    for (N, rows, dev), ent in groups.items():
        ent = ent + pads.get((N, rows, dev), [])
        Xs = []
        for _, R in ent:
            m = R.shape[1]
            if m == N:
                Xs.append(R)
                continue
            P = torch.zeros((N, N), dtype=torch.float32, device=dev)
            P[:m, :m].copy_(R)
            d = torch.arange(m, N, device=dev)
            P[d, d] = 1.0
            Xs.append(P)
        F, st, kb = be.fold_finalize_gram_batched(None, 0, Xs, 1.0 / math.sqrt(rows), damping,
                                                  out_dtype)
        for e, (key, R) in enumerate(ent):
            m = R.shape[1]
            Fe = F[e] if m == N else F[e][:m, :m].contiguous()
            out[key] = (Fe, st[e:e + 1], kb[e:e + 1])
    return out


class IFKFACRankError(RuntimeError):
    """Raised when a layer has fewer accumulated rows than columns (p < n)."""


def _module_tag(module: nn.Module) -> str:
    if isinstance(module, nn.Linear):
        return f"Linear({module.in_features}→{module.out_features})"
    if isinstance(module, nn.Conv2d):
        return f"Conv2d({module.in_channels}→{module.out_channels}, k={module.kernel_size})"
    return type(module).__name__


class RawActivationHooks(GramMatrixEstimator):
    """Streaming-TSQR factor capture for every Linear / Conv2d layer of a model.

    Parameters match the reference (activation_hooks.py:128-139).  ``math``
    selects the MFMA arithmetic of the fold (``IFKFAC`` sets bf16 when
    ``use_true_bf16`` is on).
    """

    _SEQ_SUBSAMPLE: int = 2048

    def __init__(
        self,
        model: nn.Module,
        damping: float = 1e-2,
        max_out_dim: int = 0,
        augment_bias: bool = False,
        max_conv_rows: int = 512,
        max_seq_rows: Optional[int] = None,
        batched: bool = False,
        deferred: bool = False,
        deferred_window: int = 5,
        math: int = MATH_F32,
    ):
        self.model = model
        self.damping = damping
        self.augment_bias = augment_bias
        self.max_conv_rows = max_conv_rows
        self.max_seq_rows = self._SEQ_SUBSAMPLE if max_seq_rows is None else max_seq_rows
        self.batched = batched
        self.deferred = deferred
        self.deferred_window = deferred_window
        self.math = math
        self.chunk_transform_X = None
        self.chunk_transform_G = None
        if batched and deferred:
            raise ValueError("batched and deferred modes are mutually exclusive")

        self._handles: List[torch.utils.hooks.RemovableHandle] = []
        self._enabled = False
        self._R_X: Dict[nn.Module, Optional[torch.Tensor]] = {}
        self._R_G: Dict[nn.Module, Optional[torch.Tensor]] = {}
        self._n_rows_X: Dict[nn.Module, int] = {}
        self._n_rows_G: Dict[nn.Module, int] = {}
        self._pending_X: Dict[nn.Module, List[torch.Tensor]] = {}
        self._pending_G: Dict[nn.Module, List[torch.Tensor]] = {}
        self._raw_X: Dict[nn.Module, List[torch.Tensor]] = {}
        self._raw_G: Dict[nn.Module, List[torch.Tensor]] = {}
        # persistent fold buffers (n x n fp32), reused across windows
        self._buf_X: Dict[nn.Module, torch.Tensor] = {}
        self._buf_G: Dict[nn.Module, torch.Tensor] = {}
        # Last chunk of each side held back from the fold.  An owner that
        # collects the factors and clears the hooks right after (IFKFAC's
        # factor update) sets _defer_last; the held chunk then goes straight
        # into a fused fold + finalize, one dependent factorisation instead of
        # two.  Any other reader of the running factor folds it first.
        self._defer_last = False
        self._held_X: Dict[nn.Module, Optional[torch.Tensor]] = {}
        self._held_G: Dict[nn.Module, Optional[torch.Tensor]] = {}
        # small chunks held for one larger fold (bf16 arithmetic)
        self._acc_X: Dict[nn.Module, RowAccumulator] = {}
        self._acc_G: Dict[nn.Module, RowAccumulator] = {}
        # Gram-route folds of several layers held for one batched fold per
        # shape (bf16 arithmetic)
        self._groups = FoldGroups()
        self._linear_layers: List[nn.Module] = []

        for module in model.modules():
            if not isinstance(module, (nn.Linear, nn.Conv2d)):
                continue
            if max_out_dim > 0:
                out_dim = (module.out_features if isinstance(module, nn.Linear)
                           else module.out_channels)
                if out_dim > max_out_dim:
                    continue
            self._linear_layers.append(module)
            self._R_X[module] = None
            self._R_G[module] = None
            self._n_rows_X[module] = 0
            self._n_rows_G[module] = 0
            self._pending_X[module] = []
            self._pending_G[module] = []
            self._raw_X[module] = []
            self._raw_G[module] = []
            self._held_X[module] = None
            self._held_G[module] = None
        # Gram-route folds (bf16 arithmetic) whose status the host has not
        # read: room for two batches of every factor's grouped folds
        self._fold_queue = FoldStatusQueue(cap=max(32, 4 * len(self._linear_layers)))

    # ------------------------------------------------------------------ lifecycle
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

    def clear(self):
        self._groups.discard()
        self._fold_queue.discard()
        self._acc_X.clear()
        self._acc_G.clear()
        for module in self._linear_layers:
            self._R_X[module] = None
            self._R_G[module] = None
            self._n_rows_X[module] = 0
            self._n_rows_G[module] = 0
            self._pending_X[module] = []
            self._pending_G[module] = []
            self._raw_X[module] = []
            self._raw_G[module] = []
            self._held_X[module] = None
            self._held_G[module] = None

    def remove(self):
        for h in self._handles:
            h.remove()
        self._handles.clear()
        self._enabled = False
        self.clear()
        self._buf_X.clear()
        self._buf_G.clear()

    def n_samples_accumulated(self, module: Optional[nn.Module] = None) -> int:
        target = module or (self._linear_layers[0] if self._linear_layers else None)
        if target is None:
            return 0
        return self._n_rows_X.get(target, 0)

    # ------------------------------------------------------------------ folding
    def _grouping(self) -> bool:
        return self.math == MATH_BF16 and hasattr(get_backend(), "fold_gram_batched_")

    def _flush_groups(self) -> None:
        """Fold the chunks held for grouped folds (FoldGroups)."""
        if len(self._groups):
            self._groups.flush(self.math, self._fold_queue)

    def _fold(self, side: str, module: nn.Module, chunk: torch.Tensor,
              full_rank_shape: bool = False, owned: bool = False) -> None:
        """Fold ``chunk`` into the running factor of ``module`` on ``side``
        (``owned``: the chunk is a private copy).  In bf16 arithmetic a fold by
        the Gram route is held for a grouped fold with the other layers'
        (FoldGroups); the factor view then already has its new row count."""
        if (side, module) in self._groups:
            self._flush_groups()
        Rd = self._R_X if side == "X" else self._R_G
        bufs = self._buf_X if side == "X" else self._buf_G
        n = chunk.shape[1]
        cur = Rd.get(module)
        buf = bufs.get(module)
        if buf is None or buf.shape[0] != n or buf.device != chunk.device:
            buf = torch.zeros((n, n), dtype=torch.float32, device=chunk.device)
            bufs[module] = buf
        if cur is None:
            r_in = n if full_rank_shape else 0
            if full_rank_shape:
                buf.zero_()
        else:
            r_in = cur.shape[0]
            if cur.data_ptr() != buf.data_ptr():
                buf[:r_in].copy_(cur)
        self._fold_queue.poll()
        if full_rank_shape:
            r_new = fold_chunk(buf, r_in, chunk, self.math, self._fold_queue, owned)
        else:
            acc = (self._acc_X if side == "X" else self._acc_G).setdefault(module,
                                                                            RowAccumulator())
            if self._grouping():
                # small chunks held until a fold of them pays, as the
                # accumulator does; that fold held for the grouped fold
                rows, private = acc.offer(r_in, n, chunk, owned)
                if rows is None:
                    r_new = r_in
                else:
                    if self._groups.hold((side, module), buf, r_in, rows, private):
                        self._flush_groups()
                    r_new = n
            else:
                r_new = acc.add(buf, r_in, chunk, self.math, self._fold_queue)
        Rd[module] = buf[:r_new]

    def _drain_rows(self, consume: bool, only: Optional[Tuple[str, nn.Module]] = None) -> None:
        """Fold the rows the accumulators hold -- or, with ``consume``, put them
        in front of the side's held chunk, which the fused fold + finalize
        then takes in one factorisation.  Held grouped folds go first."""
        self._flush_groups()
        for side, accs, held in (("X", self._acc_X, self._held_X),
                                 ("G", self._acc_G, self._held_G)):
            for module, acc in list(accs.items()):
                if only is not None and (side, module) != only:
                    continue
                if not acc.chunks:
                    continue
                if consume and held.get(module) is not None:
                    held[module] = torch.cat([acc.take(), held[module]], dim=0)
                    continue
                X = acc.take()
                Rd = self._R_X if side == "X" else self._R_G
                cur = Rd.get(module)
                buf = (self._buf_X if side == "X" else self._buf_G)[module]
                r_in = 0 if cur is None else cur.shape[0]
                r_new = fold_chunk(buf, r_in, X, self.math, self._fold_queue, owned=True)
                Rd[module] = buf[:r_new]

    def _finalize(self, R_raw: torch.Tensor, rows: int, out_dtype: torch.dtype,
                  math_: Optional[int] = None):
        return get_backend().finalize(R_raw, 1.0 / math.sqrt(rows), self.damping, out_dtype,
                                      self.math if math_ is None else math_)

    def _take(self, side: str, module: nn.Module, chunk: torch.Tensor) -> None:
        """Fold ``chunk``, or hold it back when the next reader is a fused finalize."""
        held = self._held_X if side == "X" else self._held_G
        prev = held.get(module)
        if prev is not None:             # chunks fold in arrival order
            self._fold(side, module, prev, owned=True)
            held[module] = None
        if not self._defer_last:
            self._fold(side, module, chunk)
            return
        # a copy: the caller may overwrite its activation or gradient in place
        held[module] = chunk.detach().clone(memory_format=torch.contiguous_format)

    def _fold_held(self) -> None:
        """Fold every held chunk into its running factor."""
        for side, held in (("X", self._held_X), ("G", self._held_G)):
            for module, chunk in held.items():
                if chunk is not None:
                    self._fold(side, module, chunk, owned=True)
                    held[module] = None

    def _running_factor(self, module: nn.Module, side: str) -> Optional[torch.Tensor]:
        """The undamped running factor of one side, held chunk folded in."""
        held = self._held_X if side == "X" else self._held_G
        chunk = held.get(module)
        if chunk is not None:
            self._fold(side, module, chunk, owned=True)
            held[module] = None
        self._drain_rows(False, (side, module))
        self._fold_queue.drain()
        return (self._R_X if side == "X" else self._R_G).get(module)

    def _side_state(self, side: str, module: nn.Module):
        """(R_raw or None, rows folded in R_raw, held chunk or None, final row count)."""
        R = (self._R_X if side == "X" else self._R_G).get(module)
        chunk = (self._held_X if side == "X" else self._held_G).get(module)
        r = 0 if R is None else R.shape[0]
        if chunk is None:
            return R, r, None, (None if R is None else R.shape[0])
        n = chunk.shape[1]
        return R, r, chunk, min(r + chunk.shape[0], n)

    def _damped(self, side: str, module: nn.Module, rows: int, out_dtype: torch.dtype,
                fast: bool = False, with_inverse: bool = False, math_: Optional[int] = None):
        """(R_damped, flag, kappa bound or None) of one side; a held chunk goes
        into a fused fold + finalize.  With ``fast`` that factorisation is the
        Gram matrix + blocked Cholesky in bf16 arithmetic (which also bounds
        kappa_2 of the factor; without a held chunk its input is the running
        factor), CholeskyQR2 outer blocks in fp32 arithmetic; its flag may
        then be 2 (see _retry_cholesky_qr).  With ``with_inverse`` the Gram
        route also forms the factor's inverse and its bf16 copies in the same
        call (a fourth value (Z, Zb, ZT), else None).  ``math_`` overrides the
        hooks' arithmetic for this factorisation."""
        R, r, chunk, _ = self._side_state(side, module)
        be = get_backend()
        am = self.math if math_ is None else math_
        gram = fast and am == MATH_BF16
        if gram and with_inverse:
            bufs = self._buf_X if side == "X" else self._buf_G
            Rs, X, r_in = ([bufs.get(module)], chunk, r) if chunk is not None else (None, R, 0)
            out, st, kb, (Z, Zb, ZT) = be.fold_finalize_gram_batched(
                Rs if r_in > 0 else None, r_in, [X], 1.0 / math.sqrt(rows), self.damping,
                out_dtype, with_inverse=True)
            return out[0], st, kb, (Z[0], Zb[0], ZT[0])
        if chunk is None:
            if gram:
                # the running factor itself is the Gram route's input (p = n rows)
                return be.fold_finalize(None, 0, R, 1.0 / math.sqrt(rows), self.damping,
                                        out_dtype, am, gram=True,
                                        with_kappa=True) + (None,)
            return self._finalize(R, rows, out_dtype, am) + (None, None)
        bufs = self._buf_X if side == "X" else self._buf_G
        res = be.fold_finalize(bufs.get(module) if r > 0 else None, r, chunk,
                               1.0 / math.sqrt(rows), self.damping, out_dtype, am,
                               cqr=fast and not gram, gram=gram, with_kappa=gram)
        return res + (None,) if gram else res + (None, None)

    def _retry_cholesky_qr(self, factors, flags, extras, then, out_dtype: torch.dtype):
        """One host read of the flags of a consuming factor update (or of
        get_factors in bf16 arithmetic): a side too
        ill-conditioned for its Gram / CholeskyQR2 factorisation (flag 2) is
        recomputed by the panel factorisation, which handles any input (and
        ``then`` run on the new factor).  That refactorisation runs in fp32
        arithmetic whatever the hooks' arithmetic: flag 2 means kappa is large,
        where the bf16 panel factor's normwise error (about 2e-3), amplified
        by kappa^2 in the solves, would leave the reference's bf16-mode result
        (an fp32 Householder factor cast to bf16, triangular.py:284,299-301,
        411-416 with ifkfac.py:292-294) far behind: measured 1.6e-1 against
        its 1.3e-2 at kappa(R) = 950."""
        mods = list(flags)
        st = torch.cat([torch.cat(flags[m]) for m in mods]).cpu()
        for i, m in enumerate(mods):
            for j, side in enumerate(("X", "G")):
                if int(st[2 * i + j]) != 2:
                    continue
                rows = self._n_rows_X[m] if side == "X" else self._n_rows_G[m]
                logger.debug("get_factors() [%s]: %s factor by the panel path",
                             _module_tag(m), side)
                R, f, kb, _ = self._damped(side, m, rows, out_dtype, fast=False, math_=MATH_F32)
                fac, fl = list(factors[m]), list(flags[m])
                fac[j], fl[j] = R, f
                factors[m], flags[m] = tuple(fac), tuple(fl)
                if then is not None:
                    ex = list(extras[m])
                    ex[j] = then(side, m, R, kb)
                    extras[m] = tuple(ex)

    # ------------------------------------------------------------------ batches
    def _side_signature(self, side: str, module: nn.Module, rows: int):
        """What must agree for two layers' sides to share a batched factor update:
        the held chunk's shape, dtype and layout, the running factor's row count,
        and the row count behind the scale."""
        R, r, chunk, _ = self._side_state(side, module)
        if chunk is None:
            return None
        return (tuple(chunk.shape), chunk.dtype, chunk.stride(), r, rows, chunk.device)

    def _batch_groups(self, eligible):
        """Groups of modules whose X sides and G sides each have one signature,
        as (modules, merged): two or more modules, or a single one whose two
        sides share a signature (a square layer); ``merged`` when the X and G
        signatures agree, so that every side of the group goes into one
        batched factor update (one chain of launches instead of one per
        side: 4096 -> 4096 at p = 8192, 4.73 -> 3.72 ms per step).  The
        backend must offer the batched factor update."""
        if not hasattr(get_backend(), "fold_finalize_gram_batched"):
            return []
        by_key: Dict[tuple, list] = {}
        for module, rows_X, rows_G, _, _, _ in eligible:
            sx = self._side_signature("X", module, rows_X)
            sg = self._side_signature("G", module, rows_G)
            if sx is None or sg is None:
                continue
            by_key.setdefault((sx, sg), []).append(module)
        return [(mods, key[0] == key[1]) for key, mods in by_key.items()
                if len(mods) >= 2 or key[0] == key[1]]

    def _damped_batch(self, entries, rows: int, out_dtype: torch.dtype, then,
                      with_inverse: bool = False):
        """_damped(fast=True) for same-signature sides, given as (side, module)
        pairs, in one batched call; per entry (R_damped, flag, then's result or
        None).  The factors are views of one (B, n, n) buffer."""
        chunks, bufs = [], []
        r = 0
        for side, m in entries:
            R, r, chunk, _ = self._side_state(side, m)
            chunks.append(chunk)
            bufs.append((self._buf_X if side == "X" else self._buf_G).get(m))
        got = get_backend().fold_finalize_gram_batched(
            bufs if r > 0 else None, r, chunks, 1.0 / math.sqrt(rows), self.damping, out_dtype,
            with_inverse=with_inverse)
        out, st, kb = got[:3]

        def follow(idx):
            res = []
            for e in idx:
                side, m = entries[e]
                R, f, k = out[e], st[e:e + 1], kb[e:e + 1]
                if then is None:
                    res.append((R, f, None))
                elif with_inverse:
                    Z, Zb, ZT = got[3]
                    res.append((R, f, then(side, m, R, k, inv=(Z[e], Zb[e], ZT[e]))))
                else:
                    res.append((R, f, then(side, m, R, k)))
            return res

        ix = [e for e, (side, _) in enumerate(entries) if side == "X"]
        ig = [e for e, (side, _) in enumerate(entries) if side == "G"]
        if then is None or not ix or not ig:
            return follow(range(len(entries)))
        # both sides in the call: each side's follow-up work (its inverse in
        # fp32 accuracy where kappa asks for it) on its own side stream
        rx, rg = run_pair(out.device, lambda: follow(ix), lambda: follow(ig))
        res = [None] * len(entries)
        for e, r_ in zip(ix + ig, rx + rg):
            res[e] = r_
        return res

    # ------------------------------------------------------------------ factors
    def get_factors(self) -> Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]]:
        """Damped factors (R_X, R_G) of every layer with enough data (fp32)."""
        factors, _, _ = self._collect_factors(torch.float32)
        return factors

    def _collect_factors(self, out_dtype: torch.dtype, consume: bool = False, then=None,
                         with_inverse: bool = False):
        """get_factors with the output dtype chosen and the finite flags returned.

        With ``consume`` the caller clears the hooks right after, so a held
        chunk goes into a fused fold + finalize and the running factor is
        left as it was (it is about to be dropped); otherwise held chunks are
        folded first, exactly as get_factors leaves them.  ``then(side,
        module, R, kappa_bound)`` runs on each side's stream right after its
        factor (kappa_bound: the Gram path's device bound of kappa_2(R), or
        None) (work
        that depends on one side only starts while the other is still being
        factored); its results come back as the third value, per module as
        (X side, G side), or None without ``then``.  With ``with_inverse`` a
        side factored by the Gram route comes with its inverse, formed by
        the same call: ``then`` is then called with ``inv=(Z, Zb, ZT)``."""
        if self.deferred:
            self._drain_deferred()
        if not consume:
            self._fold_held()
        self._drain_rows(consume)       # (held grouped folds first)
        # the Gram-route folds whose status is still on its way: a refused
        # chunk goes into its running factor by the panel path now
        self._fold_queue.drain()
        # bf16 arithmetic factors every side by the Gram route (flag 2 -> panel
        # path after one host read of the flags); fp32 arithmetic takes
        # CholeskyQR2 blocks for a consumed held chunk only
        fast = consume or self.math == MATH_BF16
        factors: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        flags: Dict[nn.Module, Tuple[torch.Tensor, torch.Tensor]] = {}
        extras: Dict[nn.Module, tuple] = {}

        want_inv = with_inverse and then is not None

        def side(s, module, rows, fast):
            R, f, kb, inv = self._damped(s, module, rows, out_dtype, fast=fast,
                                         with_inverse=want_inv)
            if then is None:
                return R, f, None
            return R, f, (then(s, module, R, kb) if inv is None
                          else then(s, module, R, kb, inv=inv))
        eligible = []
        for module in self._linear_layers:
            R_X_raw, _, chunk_X, r_X = self._side_state("X", module)
            R_G_raw, _, chunk_G, r_G = self._side_state("G", module)
            if r_X is None or r_G is None:
                continue
            rows_X = self._n_rows_X[module]
            rows_G = self._n_rows_G[module]
            n_X = (R_X_raw if R_X_raw is not None else chunk_X).shape[1]
            n_G = (R_G_raw if R_G_raw is not None else chunk_G).shape[1]
            if r_X != n_X:
                logger.debug("get_factors() [%s]: skipped — X factor partial-rank",
                             _module_tag(module))
                continue
            if r_G != n_G:
                logger.debug("get_factors() [%s]: skipped — G factor partial-rank",
                             _module_tag(module))
                continue
            if self.batched:
                if rows_X < R_X_raw.shape[1]:
                    raise IFKFACRankError(
                        f"Layer {module}: accumulated {rows_X} rows for X, "
                        f"but need >= n_in={R_X_raw.shape[1]} (batched mode).")
                if rows_G < R_G_raw.shape[1]:
                    raise IFKFACRankError(
                        f"Layer {module}: accumulated {rows_G} rows for δ, "
                        f"but need >= n_out={R_G_raw.shape[1]} (batched mode).")
            dev = (R_X_raw if R_X_raw is not None else chunk_X).device
            eligible.append((module, rows_X, rows_G, n_X, n_G, dev))
        # a consuming bf16 factor update runs same-shape layers as one batch per
        # side (ifk_fold_finalize_gram_batched: one chain of launches for all)
        groups = self._batch_groups(eligible) if (consume and self.math == MATH_BF16) else []
        batched = {m for g, _ in groups for m in g}
        for mods, merged in groups:
            module0, rows_X, rows_G, n_X, n_G, dev = next(e for e in eligible if e[0] is mods[0])
            if merged:
                # every side of the group in one batched call
                res = self._damped_batch([("X", m) for m in mods] + [("G", m) for m in mods],
                                         rows_X, out_dtype, then, want_inv)
                resX, resG = res[:len(mods)], res[len(mods):]
            else:
                resX, resG = run_pair(
                    dev,
                    lambda: self._damped_batch([("X", m) for m in mods], rows_X, out_dtype, then,
                                               want_inv),
                    lambda: self._damped_batch([("G", m) for m in mods], rows_G, out_dtype, then,
                                               want_inv),
                    b_first=n_G > n_X)
            for m, (R_X, fX, eX), (R_G, fG, eG) in zip(mods, resX, resG):
                factors[m] = (R_X, R_G)
                flags[m] = (fX, fG)
                extras[m] = (eX, eG)
        if (not consume and then is None and fast and self.math == MATH_BF16 and
                hasattr(get_backend(), "fold_finalize_gram_batched")):
            # get_factors of the running factors (no chunk held): every side
            # of every layer grouped by width (grouped_gram_finalize)
            items = []
            for module, rows_X, rows_G, _, _, _ in eligible:
                if module in batched:
                    continue
                for side, rows in (("X", rows_X), ("G", rows_G)):
                    R, _, chunk, _ = self._side_state(side, module)
                    if chunk is None and R is not None and R.shape[0] == R.shape[1]:
                        items.append(((module, side), R, rows))
            if len(items) > 1:
                got = grouped_gram_finalize(items, self.damping, out_dtype)
                for module, _, _, _, _, _ in eligible:
                    if (module, "X") in got and (module, "G") in got:
                        (R_X, fX, _), (R_G, fG, _) = got[(module, "X")], got[(module, "G")]
                        factors[module] = (R_X, R_G)
                        flags[module] = (fX, fG)
                        extras[module] = (None, None)
                        batched.add(module)
        for module, rows_X, rows_G, n_X, n_G, dev in eligible:
            if module in batched:
                continue
            # the two sides are independent: finalize them concurrently, the
            # wider (longer) one enqueued first
            (R_X, fX, eX), (R_G, fG, eG) = run_pair(
                dev,
                lambda: side("X", module, rows_X, fast),
                lambda: side("G", module, rows_G, fast),
                b_first=n_G > n_X)
            factors[module] = (R_X, R_G)
            flags[module] = (fX, fG)
            extras[module] = (eX, eG)
        if fast and flags:
            self._retry_cholesky_qr(factors, flags, extras, then, out_dtype)
        return factors, flags, (extras if then is not None else None)

    # ------------------------------------------------------------------ modes
    def _drain_deferred(self):
        for module in self._linear_layers:
            if self._raw_X.get(module):
                X = torch.cat(self._raw_X[module], dim=0)
                self._fold("X", module, X, owned=True)
                self._raw_X[module] = []
            if self._raw_G.get(module):
                G = torch.cat(self._raw_G[module], dim=0)
                self._fold("G", module, G, owned=True)
                self._raw_G[module] = []

    def flush(self):
        """Fold the chunks buffered in batched mode (no-op otherwise).

        Like the reference's bucketed flush (activation_hooks.py:370-457) the
        result is always an ``n x n`` factor: layers without data start from a
        zero factor, and zero rows contribute nothing.
        """
        if not self.batched:
            return
        self._flush_groups()
        for side, pending in (("X", self._pending_X), ("G", self._pending_G)):
            work = []
            for module in list(pending.keys()):
                chunks = pending[module]
                if not chunks:
                    continue
                X = chunks[0] if len(chunks) == 1 else torch.cat(chunks, dim=0)
                work.append((module, X))
                pending[module] = []
            # same-shape layers fold together (the reference's batched_qr over
            # a bucket, triangular.py:331-379): in bf16 arithmetic a square
            # fold by the batched Gram route, one status read for the group
            groups: Dict[tuple, list] = {}
            for module, X in work:
                key = (X.shape[0], X.shape[1], X.dtype, X.device, self._rows_in(side, module, X))
                groups.setdefault(key, []).append((module, X))
            for (p, n, _, _, r_in), items in groups.items():
                if (len(items) > 1 and self.math == MATH_BF16 and r_in + p >= n and
                        hasattr(get_backend(), "fold_gram_batched_")):
                    self._fold_group(side, items, r_in)
                else:
                    for module, X in items:
                        self._fold(side, module, X, full_rank_shape=True)

    def _rows_in(self, side: str, module: nn.Module, X: torch.Tensor) -> int:
        """The rows a flush fold of X starts from (as _fold with full_rank_shape)."""
        cur = (self._R_X if side == "X" else self._R_G).get(module)
        return X.shape[1] if cur is None else cur.shape[0]

    def _fold_group(self, side: str, items, r_in: int) -> None:
        """_fold(full_rank_shape=True) of same-shape chunks into their layers'
        running factors by one batched Gram-route fold; a layer the Gram route
        refuses (status 2, its buffer untouched) folds by the panel path once
        its status has been read (FoldStatusQueue: no host read here)."""
        Rd = self._R_X if side == "X" else self._R_G
        bufs_d = self._buf_X if side == "X" else self._buf_G
        bufs = []
        for module, X in items:
            n = X.shape[1]
            cur = Rd.get(module)
            buf = bufs_d.get(module)
            if buf is None or buf.shape[0] != n or buf.device != X.device:
                buf = torch.zeros((n, n), dtype=torch.float32, device=X.device)
                bufs_d[module] = buf
            if cur is None:
                buf.zero_()
            elif cur.data_ptr() != buf.data_ptr():
                buf[:r_in].copy_(cur)
            if r_in < n:
                buf[r_in:].zero_()
            bufs.append(buf)
        self._fold_queue.poll()
        st = get_backend().fold_gram_batched_(bufs, r_in, [X for _, X in items], GRAM_FOLD_TOL)
        for e, (module, X) in enumerate(items):
            self._fold_queue.push(st[e:e + 1], bufs[e], X, self.math)
            Rd[module] = bufs[e][:X.shape[1]]

    # ------------------------------------------------------------------ conv helpers
    @staticmethod
    def _unfold_conv_input(x: torch.Tensor, module: nn.Conv2d) -> torch.Tensor:
        x_unf = F.unfold(x, kernel_size=module.kernel_size, dilation=module.dilation,
                         padding=module.padding, stride=module.stride)
        B, C_kk, L = x_unf.shape
        return x_unf.permute(0, 2, 1).reshape(B * L, C_kk)

    @staticmethod
    def _reshape_conv_grad(delta: torch.Tensor) -> torch.Tensor:
        B, C_out, H_out, W_out = delta.shape
        return delta.permute(0, 2, 3, 1).reshape(B * H_out * W_out, C_out)

    # ------------------------------------------------------------------ hooks
    def _forward_hook(self, module: nn.Module, input: Tuple[torch.Tensor, ...],
                      output: torch.Tensor):
        if not self._enabled:
            return
        x = input[0].detach()
        if isinstance(module, nn.Conv2d):
            x = self._unfold_conv_input(x, module)
            if self.max_conv_rows > 0 and x.shape[0] > self.max_conv_rows:
                idx = torch.randperm(x.shape[0], device=x.device)[:self.max_conv_rows]
                x = x[idx]
        elif x.ndim > 2:
            x = x.reshape(-1, x.shape[-1])
            if self.max_seq_rows > 0 and x.shape[0] > self.max_seq_rows:
                idx = torch.randperm(x.shape[0], device=x.device)[:self.max_seq_rows]
                x = x[idx]
        if self.augment_bias and isinstance(module, nn.Linear) and module.bias is not None:
            ones = torch.ones(x.shape[0], 1, device=x.device, dtype=x.dtype)
            x = torch.cat([x, ones], dim=1)
        if self.chunk_transform_X is not None:
            x = self.chunk_transform_X(x)

        if self.deferred:
            self._raw_X[module].append(x)
            self._n_rows_X[module] += x.shape[0]
            if len(self._raw_X[module]) >= self.deferred_window:
                Xc = torch.cat(self._raw_X[module], dim=0)
                self._fold("X", module, Xc, owned=True)
                self._raw_X[module] = []
            return
        if self.batched:
            self._pending_X[module].append(x)
            self._n_rows_X[module] += x.shape[0]
            return
        self._take("X", module, x)
        self._n_rows_X[module] += x.shape[0]

    def _backward_hook(self, module: nn.Module, grad_input: Tuple[torch.Tensor, ...],
                       grad_output: Tuple[torch.Tensor, ...]):
        if not self._enabled:
            return
        delta = grad_output[0].detach()
        if isinstance(module, nn.Conv2d):
            delta = self._reshape_conv_grad(delta)
        elif delta.ndim > 2:
            delta = delta.reshape(-1, delta.shape[-1])
            if self.max_seq_rows > 0 and delta.shape[0] > self.max_seq_rows:
                idx = torch.randperm(delta.shape[0], device=delta.device)[:self.max_seq_rows]
                delta = delta[idx]
        if self.chunk_transform_G is not None:
            delta = self.chunk_transform_G(delta)

        if self.deferred:
            self._raw_G[module].append(delta)
            self._n_rows_G[module] += delta.shape[0]
            if len(self._raw_G[module]) >= self.deferred_window:
                Gc = torch.cat(self._raw_G[module], dim=0)
                self._fold("G", module, Gc, owned=True)
                self._raw_G[module] = []
            return
        if self.batched:
            self._pending_G[module].append(delta)
            self._n_rows_G[module] += delta.shape[0]
            return
        self._take("G", module, delta)
        self._n_rows_G[module] += delta.shape[0]
