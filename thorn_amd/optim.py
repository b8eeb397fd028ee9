"""THORN optimizer on MI355X: the reference's Python API over the HIP library.

Drop-in for ``thorn.THORN`` (pykeio/THORN, thorn/thorn.py:1229): the constructor overloads, the
parameter-group keys and defaults, the validation errors, the per-parameter state keys (and so
``state_dict``/``load_state_dict``) and ``step(closure=None, *, param=None)`` are the reference's.
What runs underneath is different: every group's whole step is a handful of grouped HIP launches
on the current stream (see ``thorn_amd.csrc``), driven through the C ABI in include/thorn_amd.h.

Magma ``momentum_align`` (thorn.py:800-836) runs without the reference's ``.item()`` host sync:
the random mask comes from the per-parameter PRNG state, a host integer as in the reference, and
the cosine-similarity EMA ``s`` stays on the device, where the kernels read it as a learning-rate
factor.

``decouple_md`` runs on orthogonalized and non-orthogonalized groups alike: the tensors of an Adam
group with it take the Adam step inside the same gain round trip as the matrices (thorn.py:1704-1721).

Not implemented on this path (each raises ``NotImplementedError`` instead of silently changing
behaviour): DTensor/FSDP2 parameters (thorn.py:979-1186, 1459-1581), a ``decouple_md`` norm axis
other than the last two dims or the last dim, dtypes other than fp32 and bf16, and a sparse
gradient on a parameter that is not contiguous fp32.
"""
from __future__ import annotations

import contextlib
import math
import weakref
from dataclasses import dataclass, field, fields, MISSING
from functools import partial
from typing import Any, Callable, Literal, Optional, Union, cast, overload

import numpy as np
import torch
import torch.nn as nn
from torch.nn import Parameter
from torch.optim import Optimizer
from typing_extensions import NotRequired, TypedDict

from . import _coeffs
from . import _lib

__all__ = ['THORN', 'THORNOrthoGroup', 'THORNNonOrthoGroup', 'THORNGroup']

# softplus(LN_E_SUB_1) == 1 (thorn.py:1602)
LN_E_SUB_1 = 0.5413248546

_TargetNorm = Union[Literal['init', 'min', 'max'], Callable[[torch.Tensor], Union[torch.Tensor, float]]]


class THORNOrthoGroup(TypedDict, total=True):
    """Keys of an orthogonalized group (thorn.py:1188-1209)."""
    orthogonalize: Literal[True]
    params: list
    lr: NotRequired[float]
    betas: NotRequired[tuple]
    weight_decay: NotRequired[float]
    none_grad: NotRequired[bool]
    scaling_mode: NotRequired[Literal['md', 'moonlight', 'jordan']]
    target_rms: NotRequired[float]
    decouple_md: NotRequired[bool]
    target_norm: NotRequired[_TargetNorm]
    gain_lr: NotRequired[float]
    gain_betas: NotRequired[tuple]
    split_gain: NotRequired[bool]
    momentum_align: NotRequired[bool]
    force_per_neuron_norm: NotRequired[bool]
    iters: NotRequired[int]
    lower_bound: NotRequired[float]
    cushion: NotRequired[float]
    safety_factor: NotRequired[float]
    coeffs: NotRequired[list]


class THORNNonOrthoGroup(TypedDict, total=True):
    """Keys of a non-orthogonalized group (thorn.py:1211-1225)."""
    orthogonalize: Literal[False]
    params: list
    lr: NotRequired[float]
    betas: NotRequired[tuple]
    weight_decay: NotRequired[float]
    none_grad: NotRequired[bool]
    rectify: NotRequired[bool]
    eps: NotRequired[float]
    momentum_align: NotRequired[bool]
    decouple_md: NotRequired[bool]
    target_norm: NotRequired[_TargetNorm]
    gain_lr: NotRequired[float]
    gain_betas: NotRequired[tuple]
    split_gain: NotRequired[bool]


THORNGroup = Union[THORNOrthoGroup, THORNNonOrthoGroup]


@dataclass
class _Group:
    """Per-step view of a parameter group: the reference's _THORNParameterGroup (thorn.py:535-612),
    rebuilt from the group dict at every step so LR schedulers take effect."""
    orthogonalize: bool
    params: list
    lr: float
    base_lr: float = field(init=False)
    none_grad: bool = field(default=True)
    weight_decay: float = field(default=0.1)
    betas: tuple = field(default_factory=lambda: (0.9, 0.95))
    scaling_mode: Optional[str] = field(default=None)
    target_rms: float = field(default=0.2)
    target_norm: Any = field(default=None)
    iters: int = field(default=5)
    rectify: bool = field(default=False)
    eps: float = field(default=0)
    lower_bound: float = field(default=1e-3)
    safety_factor: float = field(default=0.03)
    cushion: float = field(default=0.02)
    momentum_align: bool = field(default=False)
    coeffs: list = field(init=False)
    restarts: list = field(init=False)
    decouple_md: bool = field(default=False)
    gain_lr: float = field(default=1e-3)
    gain_betas: tuple = field(default_factory=lambda: (0.9, 0.95))
    norm_axis: Any = field(default=None)
    split_gain: bool = field(default=True)
    force_per_neuron_norm: bool = field(default=False)

    @classmethod
    def from_kwargs(cls, **kwargs) -> '_Group':
        return cls(**{k: kwargs[k] for k in kwargs if k in cls.__dataclass_fields__})

    def __post_init__(self):
        if self.lr < 0.0:
            raise ValueError(f'Invalid learning rate `{self.lr}`; should be >= 0')
        if not (0.0 <= self.betas[0] < 1.0):
            raise ValueError(f'Invalid beta1 `{self.betas[0]}`; should be in [0, 1)')
        if not (0.0 <= self.betas[1] < 1.0):
            raise ValueError(f'Invalid beta2 `{self.betas[1]}`; should be in [0, 1)')
        self.base_lr = self.lr
        c = _coeffs.ns_coefficients(self.lower_bound, self.iters, self.safety_factor, self.cushion)
        self.coeffs = list(c)
        self.restarts = list(_coeffs.gram_restarts(c))

    @property
    def scaling_mode_(self) -> str:
        if self.scaling_mode is None:
            return 'md' if self.decouple_md else 'moonlight'
        return self.scaling_mode

    @property
    def gain_lr_(self) -> float:
        return self.gain_lr * (float(self.lr) / self.base_lr)

    def norm_axis_(self, p: torch.Tensor):
        return self.norm_axis if self.norm_axis is not None else ((-2, -1) if p.ndim > 1 else -1)

    def target_norm_(self, p: torch.Tensor) -> torch.Tensor:
        tn = self.target_norm
        if tn is None:
            tn = 'max' if self.orthogonalize else 'init'
        if callable(tn):
            tn = tn(p)
        elif tn == 'init':
            tn = p.norm(dim=self.norm_axis_(p), keepdim=True)
        elif tn == 'min':
            tn = min(p.size(-2), p.size(-1)) ** 0.5
        elif tn == 'max':
            tn = max(p.size(-2), p.size(-1)) ** 0.5
        if isinstance(tn, (float, int)):
            return torch.full((), tn, dtype=p.dtype, device=p.device)
        return tn.to(dtype=p.dtype, device=p.device)


def _lr_scale_ortho(shape, group: _Group) -> float:
    """thorn.py:768-780."""
    rows, cols = shape[-2], shape[-1]
    mode = group.scaling_mode_
    if mode == 'md':
        return max(rows / cols, cols / rows) ** 0.5
    if mode == 'moonlight':
        assert group.target_rms > 0
        return group.target_rms * (max(1, rows, cols) ** 0.5)
    if mode == 'jordan':
        return max(1, rows / cols) ** 0.5
    raise ValueError(f'Invalid scaling_mode `{mode}`')


def _compute_rect(group: _Group, step) -> float:
    """RAdam rectification term (thorn.py:782-798)."""
    beta2 = group.betas[1]
    if beta2 > 0.0:
        rho_inf = 2 / (1 - beta2) - 1
        rho = rho_inf - 2 * step * (beta2 ** step) / (1 - beta2 ** step)
        return (
            ((rho - 4) * (rho - 2) * rho_inf / ((rho_inf - 4) * (rho_inf - 2) * rho)) ** 0.5
            if rho > 4.0 else 0.0
        ) ** float(group.rectify)
    return 1.0


def _needs_neuron_norm(shape, group: _Group) -> bool:
    """thorn.py:704-707."""
    return group.betas[1] > 0 and (shape[-2] > shape[-1] or group.force_per_neuron_norm)


_W1_C = 0xD07EBC63274654C7
_U64 = (1 << 64) - 1


def _w1rand(s: int) -> tuple[int, int]:
    """Magma's PRNG (thorn.py:800-804): a Weyl step s += C, then the xor of the high and low
    64-bit halves of the 128-bit product s * (s ^ C). Returns (new state, draw)."""
    s = (s + _W1_C) & _U64
    t = s * (s ^ _W1_C)
    return s, ((t >> 64) ^ t) & _U64


def _magma_seed(p: torch.Tensor) -> int:
    """Initial Magma PRNG state (thorn.py:1616-1619): 63 random bits from the generator of the
    parameter's device, so that torch.manual_seed fixes it as in the reference."""
    return int(torch.randint(0, (1 << 63) - 1, (), device=p.device, dtype=torch.uint64).item())


def _magma_unmasked(state: dict) -> bool:
    """Advances the parameter's PRNG; False when this step is masked (an odd draw,
    thorn.py:831-833). The new s, which scales an unmasked step, is computed on the device."""
    state['random_state'], draw = _w1rand(state['random_state'])
    return draw % 2 == 0


# Storage types of parameters, gradients and state (the reference is generic over them: its state
# takes p.dtype, thorn.py:1591-1634). Others than contiguous fp32 step through fp32 working copies
# (_Shadow) in fp32 arithmetic: bf16 and fp16 round the results to their dtype once per step (the
# reference rounds after each of its ops, and its fp16 Adam underflows g^2, 1e-6 at a 1e-3
# gradient, which fp32 does not); fp64 adds each step's fp32 change to its fp64 values, which
# keep their low-order bits.
_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float64)


def _check_tensor(t: torch.Tensor, what: str) -> None:
    if t.dtype not in _DTYPES:
        raise NotImplementedError(f'THORN on MI355X supports fp32, bf16, fp16 and fp64 tensors; {what} is {t.dtype}')
    if not t.is_cuda:
        raise RuntimeError(f'THORN on MI355X needs device tensors; {what} is on {t.device}')


def _needs_shadow(p: torch.Tensor) -> bool:
    g = p.grad
    return (p.dtype != torch.float32 or not p.is_contiguous() or
            (g is not None and not g.is_sparse and (g.dtype != torch.float32 or not g.is_contiguous())))


class _Shadow:
    """The fp32 working copy of a parameter that is not contiguous fp32 (a bf16 model, thorn.py
    README's gradient-release example; a strided view): a contiguous fp32 parameter with a gradient
    buffer and fp32 copies of the state tensors, loaded from the parameter and its state before
    the step and written back after it. The kernels then run their fp32 arithmetic; the parameter
    and its state are rounded to their own dtype once per step (the reference rounds after every
    torch op, thorn.py:1381, 1404, 702), and per-row normalization uses the dtype's eps (:720)."""

    # transposed: the working copy is p's trailing matrices transposed (a decouple_md norm over
    # dim -2 becomes one over rows); state tensors are transposed with it and the row and column
    # gains (with their moments) swap roles
    _SWAP = {'row_gain': 'col_gain', 'col_gain': 'row_gain', 'row_gain_moment': 'col_gain_moment',
             'col_gain_moment': 'row_gain_moment', 'row_gain_variance': 'col_gain_variance',
             'col_gain_variance': 'row_gain_variance'}

    def __init__(self, p: torch.Tensor, transposed: bool = False):
        self.transposed = transposed
        shape = p.mT.shape if transposed else p.shape
        self.param = torch.nn.Parameter(torch.empty(shape, dtype=torch.float32, device=p.device),
                                        requires_grad=False)
        self.param._thorn_dtype = p.dtype
        if transposed:
            self.param._thorn_md_mode = 'rows'
        self.grad = torch.empty(shape, dtype=torch.float32, device=p.device)
        self.state: dict = {}
        # fp64: the fp32 values as loaded, so that store() adds the step's change to the fp64 ones
        self.delta = p.dtype == torch.float64
        self.p0 = torch.empty_like(self.param.data) if self.delta else None
        self.state0: dict = {}

    def _key(self, k: str) -> str:
        return self._SWAP.get(k, k) if self.transposed else k

    def _view(self, t: torch.Tensor) -> torch.Tensor:
        """t in the working copy's orientation (a view)."""
        return t.mT if self.transposed and t.ndim >= 2 else t

    def reserve(self, state: dict) -> bool:
        """Allocates the fp32 copies of state tensors that have none (or another shape); True if
        it allocated any."""
        fresh = False
        for k, v in state.items():
            if not torch.is_tensor(v):
                continue
            wk, shape = self._key(k), self._view(v).shape
            if wk not in self.state or self.state[wk].shape != shape:
                self.state[wk] = torch.empty(shape, dtype=torch.float32, device=v.device)
                if self.delta:
                    self.state0[wk] = torch.empty_like(self.state[wk])
                fresh = True
        return fresh

    def load(self, p: torch.Tensor, state: dict) -> None:
        """Copies the parameter, its gradient and its state in (reserve() first)."""
        self.param.data.copy_(self._view(p.detach()))
        self.grad.copy_(self._view(p.grad))
        self.param.grad = self.grad
        if self.delta:
            self.p0.copy_(self.param.data)
        for k, v in state.items():
            wk = self._key(k)
            if torch.is_tensor(v):
                self.state[wk].copy_(self._view(v))
                if self.delta:
                    self.state0[wk].copy_(self.state[wk])
            else:
                self.state[wk] = v

    def store(self, p: torch.Tensor, state: dict) -> None:
        """Writes the step back: rounded to the dtype, or (fp64) as v + (new - loaded)."""
        with torch.no_grad():
            pv = self._view(p)
            if self.delta:
                pv.add_(self.param.data).sub_(self.p0)
            else:
                pv.copy_(self.param.data)
        for k, v in state.items():
            if torch.is_tensor(v):
                wk, vv = self._key(k), self._view(v)
                if self.delta:
                    vv.add_(self.state[wk]).sub_(self.state0[wk])
                else:
                    vv.copy_(self.state[wk])


def _matrix_view(p: torch.Tensor) -> tuple:
    """(rows, cols, batch): a parameter as a batch of rows x cols matrices over its last two dims
    (thorn.py:629, 707, 777); a vector or scalar is one 1 x n matrix."""
    if p.ndim >= 2:
        return p.shape[-2], p.shape[-1], math.prod(p.shape[:-2])
    return 1, max(1, p.numel()), 1


def _md_norm_mode(p: torch.Tensor, group: _Group) -> str:
    """decouple_md renormalization axis of a non-orthogonalized tensor (thorn.py:594-595, 1717):
    'matrix' for a norm over each trailing matrix (the default; a vector's whole length), 'rows'
    for one over each row (norm_axis = -1 on ndim >= 2), 'cols' for one over each column of the
    trailing matrices (norm_axis = -2), which steps through a transposed working copy (_Shadow)
    with the roles of its row and column gains swapped. Norms across the leading dims (matrices)
    are not implemented. A working copy reports its own mode (_thorn_md_mode)."""
    mode = getattr(p, '_thorn_md_mode', None)
    if mode is not None:
        return mode
    ax = group.norm_axis_(p)
    nd = max(p.ndim, 1)
    dims = sorted({(a % nd) for a in (ax if isinstance(ax, (tuple, list)) else (ax,))})
    if p.ndim <= 1 or dims == [nd - 2, nd - 1]:
        return 'matrix'
    if dims == [nd - 1]:
        return 'rows'
    if dims == [nd - 2]:
        return 'cols'
    raise NotImplementedError(f'decouple_md with norm_axis={ax!r} on a {p.ndim}-d tensor is not implemented '
                              'on the MI355X path (supported: the last two dims, the last dim, or dim -2)')


def _md_norm_rows(p: torch.Tensor, group: _Group) -> bool:
    """The library's per-row renormalization (THORN_MAT_NORM_ROWS) for a tensor of a
    non-orthogonalized decouple_md group (its working copy's rows for a norm over columns)."""
    return _md_norm_mode(p, group) != 'matrix'


def _plan_shapes(params: list, group: _Group, adam: bool, with_owner: bool = False):
    """rows, cols and library flags of every matrix of `params` (a parameter with ndim > 2 is one
    matrix per leading index, thorn.py:629), and with_owner: each matrix's parameter index and
    index within it."""
    rows, cols, flags, owner, sub = [], [], [], [], []
    for i, p in enumerate(params):
        r, c, batch = _matrix_view(p)
        f = 0
        if adam:
            f |= _lib.MAT_ADAM | (_lib.MAT_NORM_ROWS if _md_norm_rows(p, group) else 0)
        elif _needs_neuron_norm(p.shape, group):
            f |= _lib.MAT_PER_ROW_NORM
        if group.decouple_md:
            f |= _lib.MAT_MD if (group.split_gain and p.ndim > 1) else _lib.MAT_MD_SCALAR
        for b in range(batch):
            rows.append(r)
            cols.append(c)
            flags.append(f)
            owner.append(i)
            sub.append(b)
    return (rows, cols, flags, owner, sub) if with_owner else (rows, cols, flags)


class _TableUpload:
    """Pinned host buffers for a plan's per-step table, used in turn: a buffer is refilled only
    once the copy that last read it has run (its event). This also bounds how far the host runs
    ahead of the device: about RING steps. With a group stepping as two chains on two streams, a
    host four steps ahead (queues full of cross-stream waits) made the device's first ~10 steps
    1-3 ms slower each, and two steps ahead still varied by 0.2 ms from run to run; one step
    ahead gave the steady rate from the fourth step on, and cost the one-stream path nothing."""
    RING = 1

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.bufs = [torch.empty(max(1, nbytes), dtype=torch.uint8, pin_memory=True) for _ in range(self.RING)]
        self.views = [b.numpy()[:nbytes] for b in self.bufs]   # the same pinned bytes, for numpy
        self.events: list = [None] * self.RING
        self.i = 0
        # what the device table holds (its last upload): a table equal to it is not copied again
        # (the kernels only read the table; with fixed gradient buffers and hyperparameters a
        # plan's table repeats from step to step). numpy compares and copies these few KB in
        # about a microsecond, a tenth of what the torch calls took.
        self.last = np.empty(max(1, nbytes), dtype=np.uint8)[:nbytes]
        self.last_dst = None

    def host(self) -> torch.Tensor:
        """The next buffer, once its last copy has run (a query first: a blocking wait on an event
        long completed still cost tens of microseconds, per parameter with gradient release)."""
        ev = self.events[self.i]
        if ev is not None and not ev.query():
            ev.synchronize()
        return self.bufs[self.i]

    def upload(self, dst: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> None:
        """Copies the buffer of host() into dst on `stream`, the current stream (unless dst holds
        it)."""
        i = self.i
        view = self.views[i]
        key = (dst.data_ptr(), dst.device)
        if self.last_dst != key or not np.array_equal(view, self.last):
            dst[:self.nbytes].copy_(self.bufs[i][:self.nbytes], non_blocking=True)
            self.last[:] = view
            self.last_dst = key
        if self.events[i] is None:
            self.events[i] = torch.cuda.Event()
        self.events[i].record(stream)
        self.i = (i + 1) % self.RING


class _SharedWorkspace:
    """The workspace of the single-parameter and gradient-release window runners of a group on a
    device, one buffer per stream they run on: as large as the largest of them, zero-filled when
    allocated or grown. The library lets plans share a workspace whose steps do not overlap (a plan
    that did not step last on it takes the exact first iterate); steps on one stream never overlap,
    steps on different streams may (THORN._release_flush), so each stream has its own buffer.
    Gradient release is there to save memory: the Newton-Schulz buffers then take a workspace for
    the largest window per stream instead of one per parameter or window."""

    def __init__(self, device: torch.device):
        self.device = device
        self.bufs: dict = {}   # stream handle -> tensor

    def get(self, nbytes: int) -> torch.Tensor:
        key = torch.cuda.current_stream(self.device).cuda_stream
        t = self.bufs.get(key)
        if t is None or t.numel() < nbytes:
            t = self.bufs[key] = torch.zeros(max(1, nbytes), dtype=torch.uint8, device=self.device)
        return t


class _StatusWatch:
    """The workspace status word of a runner: set by a cluster of the small-matrix launch that
    timed out waiting for its workgroups to become resident, and kept set until read here (the
    library never clears it). Every PERIOD steps that ran the launch it is copied into a ring of
    pinned slots with an event each; completed slots are checked at the start of each step, so
    the host never waits for the device unless all slots are still in flight, and a timeout is
    reported within PERIOD steps. check(wait=True) (THORN.check_status) reads it at once. A set
    word raises RuntimeError and is cleared on the device."""
    SLOTS = 4
    PERIOD = 16

    def __init__(self, runner: '_OrthoRunner'):
        self.runner = runner
        self.host = torch.zeros(self.SLOTS, dtype=torch.int32, pin_memory=True)
        self.events = [torch.cuda.Event() for _ in range(self.SLOTS)]
        self.pending = [False] * self.SLOTS
        self.next = 0
        self.unread = 0          # steps since the last read
        self.stream = None       # the stream of the last step

    def _word(self) -> torch.Tensor:
        ws = self.runner.workspace
        return ws[_lib.WS_STATUS_OFFSET:_lib.WS_STATUS_OFFSET + 4].view(torch.int32)

    def stepped(self, stream: torch.cuda.Stream) -> None:
        """After a step that ran the small-matrix launch on stream."""
        self.stream = stream
        self.unread += 1
        if self.unread >= self.PERIOD:
            self.record()

    def record(self) -> None:
        i = self.next
        if self.pending[i]:
            self._check(i)
        with torch.cuda.stream(self.stream):
            self.host[i:i + 1].copy_(self._word(), non_blocking=True)
        self.events[i].record(self.stream)
        self.pending[i] = True
        self.next = (i + 1) % self.SLOTS
        self.unread = 0

    def check(self, wait: bool = False) -> None:
        """Raises RuntimeError if a completed read (with wait=True: a read of every step so far)
        found the word set."""
        if wait and self.unread:
            self.record()
        for k in range(self.SLOTS):
            i = (self.next + k) % self.SLOTS   # oldest first
            if self.pending[i] and (wait or self.events[i].query()):
                self._check(i)

    def _check(self, i: int) -> None:
        self.events[i].synchronize()
        self.pending[i] = False
        if int(self.host[i]) != 0:
            self.host.zero_()
            self.pending = [False] * self.SLOTS
            with torch.cuda.stream(self.stream):
                self._word().zero_()
            raise RuntimeError('THORN: the small-matrix Newton-Schulz launch timed out waiting for a '
                               'cluster of its workgroups to become resident; that step left the '
                               'parameters of its matrices with min(rows, cols) <= 256 and rows * cols '
                               '< 2^20 partly updated')


class _OrthoRunner:
    """One orthogonalized parameter set (or, with adam=True, the decouple_md tensors of a
    non-orthogonalized group, whose update is the Adam step): plan, workspace and the per-step
    table."""

    def __init__(self, params: list, group: _Group, device: torch.device, adam: bool = False,
                 workspace=None):
        self.params = params
        self.device = device
        self.adam = adam
        rows, cols, flags, owner, sub = _plan_shapes(params, group, adam, with_owner=True)
        self.rows = np.asarray(rows, dtype=np.int64)
        self.cols = np.asarray(cols, dtype=np.int64)
        self.owner = owner
        self.sub = np.asarray(sub, dtype=np.int64)
        self.plan = _lib.OrthoPlan(rows, cols, flags)
        # a tensor, a _SharedWorkspace, or None: a workspace of its own
        self.shared = workspace if isinstance(workspace, _SharedWorkspace) else None
        if self.shared is not None:
            self._ws = None
            self.shared.get(self.plan.workspace_bytes)
        else:
            self._ws = (torch.zeros(max(1, self.plan.workspace_bytes), dtype=torch.uint8, device=device)
                        if workspace is None else workspace)
        self.table = torch.empty(max(64, self.plan.table_bytes), dtype=torch.uint8, device=device)
        self.upload = _TableUpload(self.plan.table_bytes)
        self.steps = np.zeros(len(rows), dtype=_lib.ORTHO_MAT_STEP)
        self.md = group.decouple_md
        # matrices of the small-matrix launch, whose status word is read behind each step
        self.small = ((np.minimum(self.rows, self.cols) <= SMALL_MAX_S)
                      & (self.rows * self.cols < SMALL_MAX_ELEMS))
        self.status = _StatusWatch(self) if self.small.any() and not adam else None
        # per-step constants computed again only when what they depend on changes
        self._scale_key = self._eps_key = self._coeffs_key = None
        self._scale = self._eps = self._coeffs = None
        self._const_key = self._flags_key = None   # the columns weight_decay, beta1, eta, pnn_eps; step_flags
        # byte offset of each matrix in its parameter (a 3-D parameter holds several)
        self._off = (self.sub * (self.rows * self.cols) * 4).astype(np.uint64)
        # one matrix per parameter, in parameter order: the pointer columns need no gather
        self._direct = len(owner) == len(params) and list(owner) == list(range(len(params)))

    @property
    def workspace(self) -> torch.Tensor:
        return self.shared.get(self.plan.workspace_bytes) if self.shared is not None else self._ws

    def run(self, opt: 'THORN', group: _Group, unmasked: Optional[dict] = None,
            ns_begin: Optional[torch.cuda.Event] = None) -> None:
        """unmasked: id(p) -> False for a parameter whose Magma mask skips this step. ns_begin:
        recorded on the stream once the prologue launches are enqueued (thorn_ortho_step_event)."""
        params, steps = self.params, self.steps
        if self.status is not None:
            self.status.check()
        n = len(self.owner)
        elem = (self.rows * self.cols).astype(np.int64)
        bytes_off = self.sub * elem * 4
        own = self.owner
        states = [opt._state_of(p) for p in params]
        if self._direct:   # one matrix per parameter (offsets 0): the pointers as they are
            steps['p'] = [p.data_ptr() for p in params]
            steps['g'] = [p.grad.data_ptr() for p in params]
            steps['m'] = [s['moment'].data_ptr() for s in states]
        else:
            steps['p'] = np.asarray([p.data_ptr() for p in params], dtype=np.uint64)[own] + self._off
            steps['g'] = np.asarray([p.grad.data_ptr() for p in params], dtype=np.uint64)[own] + self._off
            steps['m'] = np.asarray([s['moment'].data_ptr() for s in states], dtype=np.uint64)[own] + self._off
        if self.adam:   # thorn.py:1704-1714: lr * rect, the Adam moments' scalars
            beta1, beta2 = group.betas
            st = np.asarray([s['step'] for s in states], dtype=np.float64)
            rect = np.asarray([_compute_rect(group, s['step']) for s in states], dtype=np.float64)
            steps['eta'] = (group.lr * rect)[own]
            steps['v'] = (np.asarray([s['variance'].data_ptr() for s in states], dtype=np.uint64)[own]
                          + bytes_off.astype(np.uint64))
            steps['adam_beta2'] = beta2
            steps['adam_w1'] = 1 - beta1
            steps['adam_w2'] = 1 - beta2
            steps['adam_bc1'] = (1 / (1 - beta1 ** st))[own]
            steps['adam_bc2'] = (1 / (1 - beta2 ** st))[own]
            steps['adam_eps'] = group.eps
            steps['adam_degenerate'] = (rect == 0.0).astype(np.int32)[own]
        else:
            # the group is rebuilt every step, so scaling_mode and target_rms edits take effect as
            # in the reference (thorn.py:1405); the scales depend on them and the (fixed) shapes
            skey = (group.scaling_mode_, group.target_rms)
            if self._scale_key != skey:
                self._scale = np.asarray([_lr_scale_ortho(p.shape, group) for p in params], dtype=np.float64)[own]
                self._scale_key = skey
        dts = tuple(getattr(p, '_thorn_dtype', p.dtype) for p in params)
        if self._eps_key != dts:
            self._eps = np.asarray([torch.finfo(d).eps for d in dts], dtype=np.float32)[own]
            self._eps_key = dts
        # columns that hold the same values from step to step are written when their inputs change
        ckey = (group.weight_decay, group.betas[0], None if self.adam else (group.lr, self._scale_key), dts)
        if self._const_key != ckey:
            if not self.adam:
                steps['eta'] = group.lr * self._scale
            steps['weight_decay'] = group.weight_decay
            steps['beta1'] = group.betas[0]
            steps['pnn_eps'] = self._eps
            self._const_key = ckey
        # a parameter is updated when its step is due under update_rate (thorn.py:1395); the
        # momentum (and the decouple_md round trip) runs every step
        rate = opt._update_rate
        if rate == 1 and unmasked is None:   # every parameter due
            due = np.ones(n, dtype=bool)
        else:
            due = np.asarray([(s['step'] + 1) % rate == 0 and (unmasked is None or unmasked[id(p)])
                              for p, s in zip(params, states)], dtype=bool)[own]
        keep = 0 if group.none_grad else _lib.STEP_KEEP_GRAD
        fkey = (keep, due.tobytes())
        if self._flags_key != fkey:
            steps['step_flags'] = np.where(due, _lib.STEP_APPLY | keep, keep)
            self._flags_key = fkey
        # Magma: every matrix of a parameter carries the parameter's s (thorn.py:1392, 1405)
        steps['magma_s'] = (np.asarray([s['s'].data_ptr() for s in states], dtype=np.uint64)[own]
                            if group.momentum_align else 0)
        if self.md:
            gb1, gb2 = group.gain_betas
            steps['gain_lr'] = group.gain_lr_
            steps['gain_beta2'] = gb2
            steps['gain_w1'] = 1 - gb1
            steps['gain_w2'] = 1 - gb2
            steps['gain_eps'] = group.eps
            st = np.asarray([s['step'] for s in states], dtype=np.float64)[own]
            steps['gain_bc1'] = 1 / (1 - gb1 ** st)
            steps['gain_bc2'] = 1 / (1 - gb2 ** st)
            rows = self.rows
            cols = self.cols
            sub = self.sub

            # row/column gains, or one scalar gain for vectors and split_gain=False (thorn.py:1603-1612)
            split = np.asarray(['row_gain' in s for s in states], dtype=bool)[own]

            def ptrs(key, per):
                base = np.asarray([s[key].data_ptr() if key in s else 0 for s in states], dtype=np.uint64)[own]
                return base + (sub * per * 4).astype(np.uint64)

            for name, key, per in (('row_gain', 'row_gain', rows), ('row_gain_moment', 'row_gain_moment', rows),
                                   ('row_gain_variance', 'row_gain_variance', rows),
                                   ('col_gain', 'col_gain', cols), ('col_gain_moment', 'col_gain_moment', cols),
                                   ('col_gain_variance', 'col_gain_variance', cols)):
                steps[name] = np.where(split, ptrs(key, per), np.uint64(0))
            for name, key in (('row_gain', 'gain'), ('row_gain_moment', 'gain_moment'),
                              ('row_gain_variance', 'gain_variance')):
                steps[name] = np.where(split, steps[name], ptrs(key, 0))
            # target norm: one value per matrix, or per row of each matrix (norm_axis = -1)
            tn = np.empty(n, dtype=np.uint64)
            batch = np.bincount(np.asarray(own), minlength=len(params))
            for k, (i, b) in enumerate(zip(own, sub)):
                t = states[i]['target_norm']
                per = t.numel() // batch[i] if t.numel() > 1 else 0
                tn[k] = t.data_ptr() + int(b) * per * 4
            steps['target_norm'] = tn
        host = self.upload.host()
        self.plan.fill_table(steps, self.workspace.data_ptr(), self.table.data_ptr(), host.data_ptr())
        stream = torch.cuda.current_stream(self.device)
        self.upload.upload(self.table, stream)
        ckey = (tuple(group.coeffs[:group.iters]), group.iters)
        if self._coeffs_key != ckey:
            self._coeffs = np.asarray(group.coeffs[:group.iters], dtype=np.float32).reshape(-1, 3)
            self._coeffs_key = ckey
        coeffs = self._coeffs
        if self.adam or not due.any():   # no polar factor this step: momentum (gains, Magma s) only
            coeffs = coeffs[:0]
        self.plan.step(self.table.data_ptr(), coeffs, self.restart_mask(group, coeffs.shape[0]),
                       stream.cuda_stream, ns_begin.cuda_event if ns_begin is not None else 0)
        if self.status is not None and coeffs.shape[0] and (due & self.small).any():
            self.status.stepped(stream)

    @staticmethod
    def restart_mask(group: _Group, iters: int) -> int:
        """Gram Newton-Schulz restart positions (thorn.py:582, 637-653) as a bit mask for the
        library, which runs Gram Newton-Schulz on every non-square matrix and the plain quintic on
        square ones (thorn.py:628, 654-658)."""
        return sum(1 << i for i in group.restarts if 0 < i < iters)


def _batches(params: list, limit: int) -> list:
    """Consecutive runs of parameters of at most `limit` elements each (one parameter alone when
    it is larger; limit <= 0: every parameter alone), the reference's polar_decomp_batch_size
    (thorn.py:1237, 1440) applied to a plan's parameters."""
    out, cur, n = [], [], 0
    for p in params:
        k = p.numel()
        if cur and (limit <= 0 or n + k > limit):
            out.append(cur)
            cur, n = [], 0
        cur.append(p)
        n += k
    if cur:
        out.append(cur)
    return out


def _large_matrices(params: list) -> int:
    """Matrices of `params` on the library's large-matrix path (s > 256 or r * c >= 2^20; the
    others run in its one-launch small-matrix kernel)."""
    n = 0
    for p in params:
        r, c, batch = _matrix_view(p)
        if min(r, c) > SMALL_MAX_S or r * c >= SMALL_MAX_ELEMS:
            n += batch
    return n


def _ns_cost(p) -> int:
    """A parameter's Newton-Schulz work in units of s^2 * l per matrix."""
    r, c, batch = _matrix_view(p)
    return batch * min(r, c) ** 2 * max(r, c)


def _chain_count(params: list) -> int:
    """How many chains a group of large matrices steps as: 2 while its Newton-Schulz work
    (sum of s^2 * l) is at most CHAIN_MAX_COST, else 1 (one plan). Measured on MI355X boxes, one
    process per config: the Qwen3-300M set (3.2e11) 6.82-6.85 ms with 2 chains against 7.06-7.11
    with one (3: 6.87; with the present kernels 6.58 with 2, the Adam groups beside them, against
    6.64-6.65 with 3 and 7.02 with 4); its decouple_md variant 8.86-8.89 against 9.00-9.04; the Qwen3-1.7B set
    (3.3e12) 49.9-50.1 ms with one against 50.2-52.4 with 2, 51.0-52.0 with 3 and 52.4-52.6 with 4.
    (Before the block map striped a large matrix's tiles over the XCDs, four chains filled the long
    tails its 8192 x 8192 matrix left in every launch: 53.8 against 70.2 ms.)"""
    return 2 if sum(_ns_cost(p) for p in params) <= CHAIN_MAX_COST else 1


def _split_chains(params: list, n: int) -> list:
    """The parameters dealt to n chains of about equal Newton-Schulz work: by cost (s^2 * l per
    matrix), largest first, in snake order (for two: A B B A A B ...), each chain keeping the
    group's order."""
    ranked = sorted(range(len(params)), key=lambda i: -_ns_cost(params[i]))
    chain = {}
    for k, i in enumerate(ranked):
        rnd, pos = divmod(k, n)
        chain[i] = pos if rnd % 2 == 0 else n - 1 - pos
    return [[p for i, p in enumerate(params) if chain[i] == c] for c in range(n)]


def _chain_plan(params: list, limit: int) -> Optional[list]:
    """The chains a group's orthogonalized parameters step as (_OrthoBatches), or None for one
    stream: chains need one batch under `limit` with at least CHAIN_MIN_MATRICES large-path
    matrices and at least one parameter per chain (a single 3-D parameter of many matrices is one
    plan)."""
    if len(params) < 2 or _large_matrices(params) < CHAIN_MIN_MATRICES or len(_batches(params, limit)) != 1:
        return None
    n = _chain_count(params)
    if n < 2:
        return None
    chains = _split_chains(params, n)
    return chains if all(chains) else None


# A group with at least CHAIN_MIN_MATRICES large-path matrices and at most CHAIN_MAX_COST of
# Newton-Schulz work (sum of s^2 * l) steps as two chains (_OrthoBatches, _chain_count).
CHAIN_MIN_MATRICES = 16
CHAIN_MAX_COST = 1e12
# Streams of the gradient-release steps (_release_step): with the caller's own, as many as the
# device's 4 hardware queues of a process (4 of them measured 54.8 ms on config 2's hooks, 3 41.2).
RELEASE_STREAMS = 3
RELEASE_OVERLAP = True   # False: every released step on the caller's stream, in order
# Gradient release keeps the dense gradients of a group's parameters until this many bytes of them
# are there (or backward ends) and steps them as one plan or one Adam launch: one parameter's
# Newton-Schulz launches fill only 10-48 of the device's 256 CUs. This bounds the gradient memory held back
# beyond the reference's (which drops each gradient in its hook); 0 steps each parameter alone.
RELEASE_WINDOW_BYTES = 256 << 20
# step() runs the non-orthogonalized groups on a stream of their own beside an orthogonalized group
# that steps as chains (THORN._adam_side_stream): their memory-bound launches then overlap the
# chains' GEMMs (config 2 on two MI355X boxes: 6.68-6.69 against 6.75-6.77 and 6.70-6.74 against
# 6.74-6.76 ms per step).
ADAM_OVERLAP = True


def _wait_for(home: torch.cuda.Stream) -> None:
    """The current stream of home's device waits for the work enqueued on home so far."""
    ev = torch.cuda.Event()
    ev.record(home)
    torch.cuda.current_stream(home.device).wait_event(ev)


def _window_full(grad_bytes: int) -> bool:
    """A gradient-release window holding grad_bytes of gradients steps now."""
    return grad_bytes >= RELEASE_WINDOW_BYTES
SMALL_MAX_S, SMALL_MAX_ELEMS = 256, 1 << 20   # the library's small-matrix path (thorn_abi.hip)


def _adam_beside_chains(live: list, limit: int, cache: dict) -> bool:
    """Whether step() runs the non-orthogonalized groups beside the orthogonalized ones: live is
    [(orthogonalize, parameters with a gradient)] per group. Some orthogonalized group must step as
    two chains (one batch of at least CHAIN_MIN_MATRICES large matrices, at most two chains, so
    that the caller's stream, the chains and the side stream fit the 4 hardware queues of a
    process), some non-orthogonalized group must have gradients, all of them dense. cache: (live
    parameter ids, limit) -> the chain test, which walks every matrix."""
    chained = other = False
    for ortho, ps in live:
        if ortho:
            key = (tuple(id(p) for p in ps), limit)
            c = cache.get(key)
            if c is None:
                if len(cache) > 64:
                    cache.clear()
                chains = _chain_plan(ps, limit)
                c = cache[key] = chains is not None and len(chains) <= 2
            chained = chained or c
        elif ps:
            if any(p.grad.is_sparse for p in ps):
                return False
            other = True
    return chained and other


class _OrthoBatches:
    """A group's orthogonalized parameters in batches of at most polar_decomp_batch_size elements
    (thorn.py:1237, 1440): one plan per batch, run in turn on one workspace sized for the largest,
    so the Newton-Schulz buffers of only one batch exist at a time. Plans that share a workspace
    take the exact first iterate (the library keeps the cheaper prescaled one for a plan that
    stepped last on its workspace).

    A group that is one batch with at least CHAIN_MIN_MATRICES large matrices and at most
    CHAIN_MAX_COST of work runs as two chains instead (_chain_plan, _chain_count): plans of about
    equal Newton-Schulz work, each with its own workspace (together the size of one plan's), on
    streams of the optimizer, the second starting once the first one's prologue launches are
    enqueued. The chains run out of phase, so one chain's memory-bound launches and the partly
    idle last round of tiles of each of its Newton-Schulz launches run beside the other chain's
    launches (the Qwen3-300M set: 7.07-7.11 -> 6.82-6.85 ms per step).
    The results are those of one plan bit for bit: every matrix runs the same kernels on the same
    data."""

    def __init__(self, params: list, group: _Group, device: torch.device, limit: int, adam: bool = False,
                 shared: Optional[_SharedWorkspace] = None, chain: bool = True):
        """shared: the per-stream workspace of single-parameter and gradient-release runners, used
        by every batch. chain=False: never chains (gradient release runs on the chains' streams)."""
        batches = _batches(params, limit)
        self.runners = []
        self.chained = False
        workspace = None
        chains = _chain_plan(params, limit) if chain and not adam else None
        if chains is not None:
            self.chained = True
            batches = chains
            # ns_begin[i]: recorded by chain i once its prologue is enqueued (the library records
            # it again each step; a torch event is created when first recorded)
            self.ns_begin = [torch.cuda.Event() for _ in chains[:-1]]
            for ev in self.ns_begin:
                ev.record(torch.cuda.current_stream(device))
            self.fork = torch.cuda.Event()
            self.joins = [torch.cuda.Event() for _ in chains]
        elif shared is not None:   # batches, if several, run in turn on the stream's shared buffer
            workspace = shared
        elif len(batches) > 1:
            sizes = [_lib.OrthoPlan(*_plan_shapes(b, group, adam)).workspace_bytes for b in batches]
            workspace = torch.zeros(max(1, max(sizes)), dtype=torch.uint8, device=device)
        for b in batches:
            self.runners.append(_OrthoRunner(b, group, device, adam, workspace))

    @property
    def workspace_bytes(self) -> int:
        return sum({ws.data_ptr(): ws.numel() for ws in self.workspaces}.values())

    @property
    def plans(self) -> list:
        return [r.plan for r in self.runners]

    @property
    def workspaces(self) -> list:
        return [r.workspace for r in self.runners]

    def run(self, opt: 'THORN', group: _Group, unmasked: Optional[dict] = None) -> None:
        if not self.chained:
            for r in self.runners:
                r.run(opt, group, unmasked)
            return
        dev = self.runners[0].device
        main = torch.cuda.current_stream(dev)
        streams = opt._chain_streams(dev, len(self.runners))
        self.fork.record(main)            # gradients and state as the caller left them
        for i, (r, st) in enumerate(zip(self.runners, streams)):
            st.wait_event(self.fork)
            if i > 0:
                st.wait_event(self.ns_begin[i - 1])   # the previous chain's prologue is done
            with torch.cuda.stream(st):
                r.run(opt, group, unmasked, ns_begin=self.ns_begin[i] if i < len(self.ns_begin) else None)
        for ev, st in zip(self.joins, streams):    # before anything else of the step reads the results
            ev.record(st)
            main.wait_event(ev)


class _AdamBatch:
    """The plain Adam tensors of every non-orthogonalized group of one step, per device, and the
    rest of those groups' step (working-copy write-back, step counts), run after the launch."""

    def __init__(self):
        self.entries: dict = {}
        self.finish: list = []


class _AdamRunner:
    """All tensors of the non-orthogonalized groups of one step: one multi-tensor launch."""

    def __init__(self, params: list, device: torch.device):
        self.params = params
        self.device = device
        self.plan = _lib.AdamPlan([p.numel() for p in params])
        self.table = torch.empty(max(64, self.plan.table_bytes), dtype=torch.uint8, device=device)
        self.upload = _TableUpload(self.plan.table_bytes)
        self.workspace = torch.empty(max(256, self.plan.workspace_bytes), dtype=torch.uint8, device=device)
        self.steps = np.zeros(len(params), dtype=_lib.ADAM_TENSOR_STEP)
        self.memo: dict = {}   # _fill_adam_steps: the hyperparameter columns of the last step

    @property
    def plans(self) -> list:
        return [self.plan]

    @property
    def workspaces(self) -> list:
        return [self.workspace]

    def run(self, entries: list, update_rate: int = 1) -> None:
        """entries: (p, state, group, unmasked) per tensor, in plan order, from any number of
        groups. A tensor's parameter is written only when its step is due under update_rate
        (thorn.py:1706-1707) and not masked by Magma (unmasked False); m and v always are."""
        _fill_adam_steps(self.steps, entries, update_rate, self.memo)
        host = self.upload.host()
        self.plan.fill_table(self.steps, self.workspace.data_ptr(), self.table.data_ptr(), host.data_ptr())
        stream = torch.cuda.current_stream(self.device)
        self.upload.upload(self.table, stream)
        self.plan.step(self.table.data_ptr(), stream.cuda_stream)


def _fill_adam_steps(s: np.ndarray, entries: list, update_rate: int, memo: dict) -> None:
    """The per-step records of an Adam launch (ADAM_TENSOR_STEP) from entries (p, state, group,
    unmasked). Entries come group by group, and within a run of entries of one group object with
    one step count every scalar is the same: computed once and written to the run's slice (the
    hyperparameter columns only when they differ from the last call's, kept in memo), with the
    same Python arithmetic per value as per entry. Values are those of the per-entry form."""
    n = len(entries)
    s['p'] = [e[0].data_ptr() for e in entries]
    s['g'] = [e[0].grad.data_ptr() for e in entries]
    s['m'] = [e[1]['moment'].data_ptr() for e in entries]
    s['v'] = [e[1]['variance'].data_ptr() for e in entries]
    steps = [e[1]['step'] for e in entries]
    runs = []
    i = 0
    while i < n:
        grp, st = entries[i][2], steps[i]
        j = i + 1
        while j < n and entries[j][2] is grp and steps[j] == st:
            j += 1
        runs.append((i, j, grp, st))
        i = j
    hyper = tuple((i, j, g.weight_decay, g.betas[1], g.betas[0], g.eps) for i, j, g, _ in runs)
    if memo.get('hyper') != hyper:
        for i, j, g, _ in runs:
            s['weight_decay'][i:j] = g.weight_decay
            s['beta2'][i:j] = g.betas[1]
            s['w1'][i:j] = 1 - g.betas[0]
            s['w2'][i:j] = 1 - g.betas[1]
            s['eps'][i:j] = g.eps
        memo['hyper'] = hyper
    for i, j, g, st in runs:
        r = _compute_rect(g, st)
        s['lr'][i:j] = g.lr * r * 1.0
        s['bc1'][i:j] = 1 / (1 - g.betas[0] ** st)
        s['bc2'][i:j] = 1 / (1 - g.betas[1] ** st)
        s['degenerate'][i:j] = 1 if r == 0.0 else 0
        due = (st + 1) % update_rate == 0
        if g.momentum_align:
            s['apply'][i:j] = [1 if due and e[3] else 0 for e in entries[i:j]]
            s['magma_s'][i:j] = [e[1]['s'].data_ptr() for e in entries[i:j]]
        else:
            s['apply'][i:j] = 1 if due else 0
            s['magma_s'][i:j] = 0


class THORN(Optimizer):
    """Drop-in for pykeio/THORN's ``THORN`` (thorn.py:1229-1776) on one MI355X."""

    param_groups: list
    # Elements of the parameters whose Newton-Schulz runs in one batch (thorn.py:1237, 1440): a
    # group's orthogonalized parameters are planned in consecutive batches of at most this many
    # elements (0: one parameter per batch), run in turn on one workspace. The reference's default
    # is 32 Mi elements; here it is 2 Gi, so that a group is one batch on a 288 GB MI355X: the
    # grouped launches over all of a group's matrices are what fills the GPU.
    polar_decomp_batch_size: int = 2 * 1024 * 1024 * 1024

    @overload
    def __init__(self, params: nn.Module, *, lr: float, none_grad: bool = True, weight_decay: float = 0.1,
                 betas: tuple = (0.9, 0.95), scaling_mode: Optional[str] = None, target_rms: float = 0.2,
                 target_norm: Optional[_TargetNorm] = None, iters: int = 5, rectify: bool = False,
                 eps: float = 0, lower_bound: float = 1e-3, safety_factor: float = 0.03,
                 cushion: float = 0.02, momentum_align: bool = False, gradient_release: bool = False,
                 decouple_md: bool = False, gain_lr: float = 1e-3, gain_betas: tuple = (0.9, 0.95),
                 split_gain: bool = True, backend=torch.cuda): ...

    @overload
    def __init__(self, params: list): ...

    def __init__(self, params, *, backend=torch.cuda, **conf):
        _lib.load()   # fail at construction, not at the first step, when the library is missing
        self._update_rate = 1
        self._shadows: dict = {}         # id(parameter) -> _Shadow, dropped with the parameter
        self._shadow_state: dict = {}    # id(shadow parameter) -> its fp32 state
        self.backend = backend
        groups = THORN._auto_assign(params, **conf) if isinstance(params, nn.Module) else params
        for group in groups:
            assert 'orthogonalize' in group
            if group['orthogonalize']:
                assert all(map(lambda x: x.ndim >= 2, group['params'])), \
                    'Only parameters with ndim >= 2 can be orthogonalized'
        self.is_distributed = False
        self.rank = None
        defaults = dict()
        for f in fields(_Group):
            if f.default is not MISSING:
                defaults[f.name] = f.default
            elif f.default_factory is not MISSING:
                defaults[f.name] = f.default_factory()
        super().__init__(cast(list, groups), defaults)
        self._param_to_group: dict = {}
        for group in self.param_groups:
            for p in group['params']:
                self._param_to_group[id(p)] = group
        self._runners: dict = {}
        self._magma_scratch: dict = {}
        self._side_streams: dict = {}
        self._adam_streams: dict = {}   # device -> the non-orthogonalized groups' stream in step()
        self._adam_events: dict = {}    # device -> (fork, join) events of that stream
        self._chains_two: dict = {}     # (live parameter ids, batch limit) -> steps as 2 chains
        self._shared_ws: dict = {}   # (group index, device) -> _SharedWorkspace
        self._release_pending: dict = {}   # device -> streams with released steps not joined yet
        self._release_events: dict = {}    # device -> the fork event and one join event per stream
        self._release_next = 0
        self._release_queued = False   # a join is queued for the end of the current backward pass
        # (group index, device) -> [stream, [(parameter, gradient)], gradient bytes]: a window not
        # stepped yet
        self._release_windows: dict = {}
        self._release_task = -1   # the autograd graph task that queued the pending join
        if isinstance(params, nn.Module) and conf.get('gradient_release', False):
            self.setup_gradient_release(params)

    @staticmethod
    def _auto_assign(module: nn.Module, **keys) -> list:
        """thorn.py:1302-1331: ndim >= 2, not an ``lm_head``, not an ``nn.Embedding`` weight."""
        embedding_params = []

        def filter_embeddings(m: nn.Module):
            if isinstance(m, nn.Embedding):
                embedding_params.append(id(m.weight))
        module.apply(filter_embeddings)
        ortho, regular = [], []
        for name, prm in module.named_parameters():
            if prm.ndim >= 2 and 'lm_head' not in name and id(prm) not in embedding_params:
                ortho.append(prm)
            else:
                regular.append(prm)
        return [{'orthogonalize': True, 'params': ortho, **keys},
                {'orthogonalize': False, 'params': regular, **keys}]

    # -- state initialisation (thorn.py:1591-1634) ---------------------------------------------
    def _init_state(self, p: torch.Tensor, group: _Group) -> None:
        state = self.state[p]
        if 'step' in state:
            return
        state['step'] = 1
        state['moment'] = torch.zeros_like(p)
        if not group.orthogonalize:
            state['variance'] = torch.zeros_like(p)
        if group.decouple_md:
            if p.ndim > 1 and group.split_gain:
                state['row_gain'] = torch.full((*p.shape[:-1], 1), LN_E_SUB_1, dtype=p.dtype, device=p.device)
                state['col_gain'] = torch.full((*p.shape[:-2], 1, *p.shape[-1:]), LN_E_SUB_1, dtype=p.dtype,
                                               device=p.device)
                for k in ['row_gain', 'col_gain']:
                    state[f'{k}_moment'] = torch.zeros_like(state[k])
                    state[f'{k}_variance'] = torch.zeros_like(state[k])
            else:
                state['gain'] = torch.full((), LN_E_SUB_1, dtype=p.dtype, device=p.device)
                state['gain_moment'] = torch.zeros((), dtype=p.dtype, device=p.device)
                state['gain_variance'] = torch.zeros((), dtype=p.dtype, device=p.device)
            state['target_norm'] = group.target_norm_(p)
        if group.momentum_align:
            state['random_state'] = _magma_seed(p)
            state['s'] = torch.ones((), dtype=p.dtype, device=p.device)

    def _validate(self, p: torch.Tensor, group: _Group) -> None:
        g = p.grad
        if group.decouple_md and not group.orthogonalize:
            _md_norm_rows(p, group)   # raises for an unsupported norm axis
        if g.is_sparse and group.orthogonalize:
            # the reference's momentum step g + beta1 * m (thorn.py:1381) fails the same way
            raise RuntimeError('add(sparse, dense) is not supported: an orthogonalized parameter needs a '
                               'dense gradient')
        if ((type(p) is not torch.nn.Parameter and type(p) is not torch.Tensor and type(p.data).__name__ == 'DTensor')
                or type(g).__name__ == 'DTensor'):
            raise NotImplementedError('DTensor / FSDP2 parameters are not implemented on the MI355X path')
        if g.shape != p.shape:
            raise AssertionError(f'gradient shape {tuple(g.shape)} != parameter shape {tuple(p.shape)}')
        _check_tensor(p, 'parameter')
        _check_tensor(g, 'gradient')
        if g.device != p.device:
            raise RuntimeError('gradient and parameter are on different devices')

    def _sparse_adam(self, p: torch.Tensor, g: torch.Tensor, group: _Group, unmasked: bool = True) -> None:
        """Row-sparse Adam on the coalesced gradient g (thorn.py:1673-1700): the gradient's rows
        of p, m and v take the ordinary Adam step (thorn_adam_sparse_step); the other rows keep
        their parameter and state. With Magma, s moves from the gradient rows and the gathered
        moment rows, and a masked step updates m and v only."""
        state = self.state[p]
        step = state['step']
        beta1, beta2 = group.betas
        rect = _compute_rect(group, step)
        rows = p.shape[0]
        row_len = p.numel() // rows if rows else 0
        idx = g.indices()[0].contiguous()
        vals = g.values().reshape(idx.numel(), row_len).contiguous()
        # a parameter (or state) that is not contiguous fp32 steps through fp32 copies of the
        # gradient's rows (the rows 0 .. nnz-1 of a compact parameter), written back rounded to its
        # dtype (fp64: as its value plus the fp32 change); the other rows are not touched
        direct = all(t.dtype == torch.float32 and t.is_contiguous()
                     for t in (p, state['moment'], state['variance'], vals))
        if direct:
            tp, tm, tv, trows, tvals = p, state['moment'], state['variance'], idx, vals
        else:
            def rows_of(t):
                return t.detach().index_select(0, idx).reshape(idx.numel(), row_len).float()
            tp, tm, tv = rows_of(p), rows_of(state['moment']), rows_of(state['variance'])
            before = [t.clone() for t in (tp, tm, tv)] if p.dtype == torch.float64 else None
            trows = torch.arange(idx.numel(), device=idx.device, dtype=idx.dtype)
            tvals = vals.float()
        rec = np.zeros(1, dtype=_lib.ADAM_SPARSE_STEP)
        rec['p'] = tp.data_ptr()
        rec['m'] = tm.data_ptr()
        rec['v'] = tv.data_ptr()
        rec['g_values'] = tvals.data_ptr()
        rec['g_rows'] = trows.data_ptr()
        rec['rows'] = tp.shape[0]
        rec['row_len'] = row_len
        rec['nnz'] = idx.numel()
        rec['lr'] = group.lr * rect * 1.0
        rec['weight_decay'] = group.weight_decay
        rec['beta2'] = beta2
        rec['w1'] = 1 - beta1
        rec['w2'] = 1 - beta2
        rec['bc1'] = 1 / (1 - beta1 ** step)
        rec['bc2'] = 1 / (1 - beta2 ** step)
        rec['eps'] = group.eps
        rec['apply'] = 1 if (step + 1) % self._update_rate == 0 and unmasked else 0
        rec['degenerate'] = 1 if rect == 0.0 else 0
        s32 = None
        if group.momentum_align:
            s32 = state['s'] if state['s'].dtype == torch.float32 else state['s'].float()
            rec['magma_s'] = s32.data_ptr()
            rec['magma_work'] = self._magma_work(p.device).data_ptr()
        with torch.cuda.device(p.device):
            _lib.adam_sparse_step(rec, torch.cuda.current_stream(p.device).cuda_stream)
        if s32 is not None and s32 is not state['s']:
            state['s'].copy_(s32)
        if not direct:
            with torch.no_grad():
                for i, (dst, new) in enumerate(((p, tp), (state['moment'], tm), (state['variance'], tv))):
                    shape = (idx.numel(), *dst.shape[1:])
                    if before is not None:   # fp64: the row values plus the fp32 change
                        new = dst.index_select(0, idx) + (new - before[i]).double().reshape(shape)
                    dst.index_copy_(0, idx, new.reshape(shape).to(dst.dtype))

    def _magma_work(self, dev: torch.device) -> torch.Tensor:
        """Device scratch of the sparse Magma statistics (one per device; steps on one stream)."""
        w = self._magma_scratch.get(dev)
        if w is None:
            w = torch.empty(_lib.SPARSE_MAGMA_WORK_BYTES, dtype=torch.uint8, device=dev)
            self._magma_scratch[dev] = w
        return w

    # Runners (plan + workspace) kept per group and device: a new set of live parameters (some
    # without a gradient this step) builds a new runner, and the least recently used one beyond
    # this many is dropped with its workspace, so memory stays bounded when the set changes.
    # Runners of a single parameter and those of gradient release's windows are kept apart, one per
    # parameter of the group at most: they share one workspace per stream, and rebuilding one per
    # call would allocate a table and a pinned buffer each time.
    _RUNNERS_PER_GROUP = 2

    def _chain_streams(self, dev: torch.device, n: int) -> tuple:
        """The n streams of a chained group on `dev` (default priority), taken one after the
        other from torch's stream pool. The runtime maps streams to the device's hardware queues in
        turn, so the two get different queues; a chain on the caller's stream could share its
        queue with the other chain's stream and run serialized behind it (measured: 7.3-7.5
        against 6.8 ms per step on config 2)."""
        s = self._side_streams.setdefault(dev, [])
        while len(s) < n:
            s.append(torch.cuda.Stream(dev))
        return tuple(s[:n])

    def _adam_side_stream(self) -> Optional[torch.cuda.Stream]:
        """The stream step() runs the non-orthogonalized groups on, beside the caller's stream with
        the orthogonalized ones, or None: every group in order on the caller's stream. A side stream
        only pays beside an orthogonalized group that steps as chains (a Newton-Schulz block fills a
        CU, so memory-bound blocks only displace the GEMMs of one plan, and on small groups the
        events cost more than the overlap gives), and only with at most two chains, so that the
        caller's stream, the chains and this one use the 4 hardware queues of a process. All
        gradients on one device, those of the non-orthogonalized groups dense."""
        if not ADAM_OVERLAP:
            return None
        live = [(g['orthogonalize'], [p for p in g['params'] if p.grad is not None]) for g in self.param_groups]
        if not _adam_beside_chains(live, int(self.polar_decomp_batch_size), self._chains_two):
            return None
        devs = {p.device for _, ps in live for p in ps}
        if len(devs) != 1:
            return None
        dev = devs.pop()
        if dev.type != 'cuda':
            return None
        st = self._adam_streams.get(dev)
        if st is None:
            st = self._adam_streams[dev] = torch.cuda.Stream(dev)
            self._adam_events[dev] = (torch.cuda.Event(), torch.cuda.Event())
        return st

    def _shared_workspace(self, gi: int, dev: torch.device) -> _SharedWorkspace:
        w = self._shared_ws.get((gi, dev))
        if w is None:
            w = self._shared_ws[(gi, dev)] = _SharedWorkspace(dev)
        return w

    def _runner(self, key, factory):
        """The runner of key = (kind, group index, device, parameter ids, ...), built by factory()
        if it is not kept."""
        r = self._runners.pop(key, None)
        if r is None:
            per_param = lambda k: len(k[3]) == 1 or k[0] == 'release'
            slot, single = key[:3], per_param(key)
            # key[1] < 0: the one Adam launch of a whole step, over every non-orthogonalized group
            cap = (len(self.param_groups[key[1]]['params']) if single and key[1] >= 0
                   else self._RUNNERS_PER_GROUP)
            same = [k for k in self._runners if k[:3] == slot and per_param(k) == single]
            for k in same[:max(0, len(same) - cap + 1)]:
                self._check_status(self._runners.pop(k))
            r = factory()
        self._runners[key] = r   # most recently used last
        return r

    # -- step (thorn.py:1583-1753) ---------------------------------------------------------------
    def _step_params(self, params: list, group: _Group, gi: int, release: bool = False,
                     adam: Optional['_AdamBatch'] = None, home: Optional[torch.cuda.Stream] = None) -> None:
        """release: a gradient-release window of large orthogonalized parameters (_release_flush),
        one plan on the current stream's shared workspace, never chained. adam: the step's batch
        of plain Adam tensors; a non-orthogonalized group without decouple_md adds its dense
        tensors to it (and the rest of their step, after the launch) instead of launching.
        home: the caller's stream when this runs on another one (the Adam side stream, a release
        stream). New optimizer state and working copies are allocated and initialized there, so
        the caching allocator ties them to the stream every other one joins back into, and the
        current stream waits for that initialization."""
        live = []
        sparse = []
        fresh = False   # state or working copies were made on `home` in this call
        for p in params:
            if p is None or p.grad is None:
                continue
            self._validate(p, group)
            if home is not None and 'step' not in self.state[p]:
                with torch.cuda.stream(home):
                    self._init_state(p, group)
                fresh = True
            else:
                self._init_state(p, group)
            g = p.grad
            if g.is_sparse and not group.orthogonalize:
                if group.decouple_md or g.sparse_dim() != 1:   # thorn.py:1671-1672
                    p.grad = g.to_dense()
                else:
                    g = g.coalesce()
                    if g.indices().numel() == 0:   # thorn.py:1677-1678: no step for this one
                        continue
                    sparse.append((p, g))
                    continue
            live.append(p)
        if fresh and home is not None:
            _wait_for(home)
            fresh = False
        # Magma masks, one PRNG draw per parameter that steps (thorn.py:1392, 1679, 1702)
        unmasked = None
        if group.momentum_align:
            unmasked = {id(p): _magma_unmasked(self.state[p]) for p in live + [q for q, _ in sparse]}
        for p, g in sparse:
            self._sparse_adam(p, g, group, True if unmasked is None else unmasked[id(p)])
        for p, _ in sparse:
            if group.none_grad:
                p.grad = None
            self.state[p]['step'] += 1
        if not live:
            return
        # parameters that are not contiguous fp32 step through their fp32 working copies
        shadows = {}
        for p in live:
            # a decouple_md norm over dim -2 of an Adam group's tensor: a transposed working copy
            tr = group.decouple_md and not group.orthogonalize and _md_norm_mode(p, group) == 'cols'
            if tr or _needs_shadow(p):
                sh = self._shadows.get(id(p))
                with torch.cuda.stream(home) if home is not None else contextlib.nullcontext():
                    if sh is None or sh.transposed != tr or sh.param.shape != (p.mT.shape if tr else p.shape):
                        if sh is None:
                            weakref.finalize(p, self._drop_shadow, id(p))
                        else:
                            self._shadow_state.pop(id(sh.param), None)
                        sh = self._shadows[id(p)] = _Shadow(p, transposed=tr)
                        self._shadow_state[id(sh.param)] = sh.state
                        fresh = True
                    fresh = sh.reserve(self.state[p]) or fresh
                shadows[p] = sh
        if fresh and home is not None:
            _wait_for(home)
        for p, sh in shadows.items():
            sh.load(p, self.state[p])
            if unmasked is not None:
                unmasked[id(sh.param)] = unmasked[id(p)]
        by_dev: dict = {}
        for p in live:
            by_dev.setdefault(p.device, []).append(shadows[p].param if p in shadows else p)
        for dev, ps in by_dev.items():
            with torch.cuda.device(dev):
                if group.orthogonalize:
                    limit = int(self.polar_decomp_batch_size)
                    key = ('release' if release else 'ortho', gi, dev, tuple(id(p) for p in ps),
                           tuple(tuple(p.shape) for p in ps), group.decouple_md, group.split_gain,
                           group.force_per_neuron_norm, group.betas[1] > 0, limit)
                    shared = self._shared_workspace(gi, dev) if len(ps) == 1 or release else None
                    runner = self._runner(key, lambda: _OrthoBatches(ps, group, dev, limit, shared=shared,
                                                                     chain=not release))
                    runner.run(self, group, unmasked)
                elif group.decouple_md:   # Adam step inside the decouple_md round trip (thorn.py:1704-1721)
                    limit = int(self.polar_decomp_batch_size)
                    key = ('mdadam', gi, dev, tuple(id(p) for p in ps), tuple(tuple(p.shape) for p in ps),
                           group.split_gain, tuple(_md_norm_rows(p, group) for p in ps), limit)
                    shared = self._shared_workspace(gi, dev) if len(ps) == 1 else None
                    runner = self._runner(key, lambda: _OrthoBatches(ps, group, dev, limit, adam=True, shared=shared))
                    runner.run(self, group, unmasked)
                else:
                    entries = [(p, self._state_of(p), group,
                                True if unmasked is None else unmasked[id(p)]) for p in ps]
                    if adam is not None:
                        adam.entries.setdefault(dev, []).extend(entries)
                    else:
                        self._adam_launch(gi, dev, entries)

        def finish():
            for p, sh in shadows.items():
                sh.store(p, self.state[p])
            for p in live:
                if group.none_grad:
                    p.grad = None
                self.state[p]['step'] += 1

        if adam is not None and not group.orthogonalize and not group.decouple_md:
            adam.finish.append(finish)
        else:
            finish()

    def _adam_launch(self, gi: int, dev: torch.device, entries: list) -> None:
        """One multi-tensor Adam launch over entries (p, state, group, unmasked); gi < 0: the
        batch of a whole step."""
        ps = [e[0] for e in entries]
        key = ('adam', gi, dev, tuple(id(p) for p in ps), tuple(p.numel() for p in ps))
        runner = self._runner(key, lambda: _AdamRunner(ps, dev))
        runner.run(entries, self._update_rate)

    def _adam_flush(self, adam: '_AdamBatch') -> None:
        """The step's one Adam launch per device, then the rest of those groups' step."""
        try:
            for dev, entries in adam.entries.items():
                with torch.cuda.device(dev):
                    self._adam_launch(-1, dev, entries)
        finally:
            for f in adam.finish:
                f()
            adam.entries.clear()
            adam.finish.clear()

    def _drop_shadow(self, key: int) -> None:
        sh = self._shadows.pop(key, None)
        if sh is not None:
            self._shadow_state.pop(id(sh.param), None)

    def _state_of(self, p: torch.Tensor) -> dict:
        """The state a runner reads: a working copy's (_Shadow), or the parameter's own."""
        st = self._shadow_state.get(id(p))
        return st if st is not None else self.state[p]

    @overload
    def step(self, closure: None = None, *, param: Optional[torch.nn.Parameter] = None) -> None: ...

    @overload
    def step(self, closure: Callable[[], float], *, param: Optional[torch.nn.Parameter] = None) -> float: ...

    @torch.no_grad()
    def step(self, closure: Optional[Callable[[], float]] = None, *, param: Optional[torch.nn.Parameter] = None):
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError('THORN.step cannot be captured in a CUDA/HIP graph: every step fills its launch '
                               'tables on the host and uploads them from pinned memory')
        self._release_recover()
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if param is None:
            # the plain Adam tensors of every non-orthogonalized group: one launch per device,
            # after the groups before a group that raises (in order: it stops the later ones)
            adam = _AdamBatch()
            side = self._adam_side_stream()
            if side is None:
                try:
                    for gi, group in enumerate(self.param_groups):
                        self._step_params(group['params'], _Group.from_kwargs(**group), gi, adam=adam)
                finally:
                    self._adam_flush(adam)
            else:
                main = torch.cuda.current_stream(side.device)
                fork, join = self._adam_events[side.device]
                fork.record(main)   # gradients and state as the caller left them
                side.wait_event(fork)
                try:
                    for gi, group in enumerate(self.param_groups):
                        if group['orthogonalize']:
                            self._step_params(group['params'], _Group.from_kwargs(**group), gi)
                            continue
                        grads = [p.grad for p in group['params'] if p.grad is not None]
                        with torch.cuda.stream(side):
                            self._step_params(group['params'], _Group.from_kwargs(**group), gi, adam=adam,
                                              home=main)
                        for g in grads:
                            g.record_stream(side)   # the step may drop them; the stream still reads them
                finally:
                    try:
                        with torch.cuda.stream(side):
                            self._adam_flush(adam)
                    finally:
                        join.record(side)
                        main.wait_event(join)
        else:
            group = self._param_to_group[id(param)]
            gi = next(i for i, g in enumerate(self.param_groups) if g is group)
            self._step_params([param], _Group.from_kwargs(**group), gi)
        return loss

    def check_status(self) -> None:
        """Waits for the steps enqueued so far and raises RuntimeError if one of them had its
        small-matrix Newton-Schulz launch time out (step() makes the same check without waiting,
        for the steps already completed, when it starts)."""
        for r in list(self._runners.values()):
            self._check_status(r)

    @staticmethod
    def _check_status(r) -> None:
        for x in getattr(r, 'runners', ()):
            if x.status is not None:
                x.status.check(wait=True)

    def _release_step(self, p: torch.Tensor, join_later: bool) -> None:
        """step(param=p) as gradient release runs it, with p.grad as it is now; the caller may drop
        p.grad afterwards (a window keeps the tensor).

        The Newton-Schulz launches of one matrix fill only a few of the device's CUs, and the
        parameters' steps are independent, so an orthogonalized parameter joins its group's window
        with its gradient: once the window holds RELEASE_WINDOW_BYTES of gradients it steps as one
        plan on the next of RELEASE_STREAMS streams (_release_flush), and the caller's stream waits
        for it in _release_join, which also steps what the windows still hold. Small matrices (the
        library's small-matrix path) and the tensors of non-orthogonalized groups join their
        group's window too: a window of them is one launch (the small-matrix step, or one
        multi-tensor Adam launch), where each would otherwise be a launch and a host round of its
        own. join_later=False steps and joins at once. A sparse gradient steps on the caller's
        stream at once."""
        group = self._param_to_group[id(p)]
        if not RELEASE_OVERLAP or not p.is_cuda or p.grad is None or p.grad.is_sparse:
            self.step(param=p)
            return
        gi = next(i for i, g in enumerate(self.param_groups) if g is group)
        key = (gi, p.device)
        cur = torch.cuda.current_stream(p.device)
        w = self._release_windows.get(key)
        if w is not None and (w[0] != cur or any(q is p for q, _ in w[1])):
            self._release_flush(key)   # a window holds gradients of one stream, each parameter once
            w = None
        if w is None:
            w = self._release_windows[key] = [cur, [], 0]
        g = p.grad
        w[1].append((p, g))
        w[2] += g.numel() * g.element_size()
        if not join_later or _window_full(w[2]):
            self._release_flush(key)
        if not join_later:
            self._release_join()

    def _release_flush(self, key) -> None:
        """Step the parameters of window `key` with the gradients it holds, as one plan on the next
        release stream, after the work their gradients' stream holds now; each parameter's .grad is
        left as it was before (None after its hook). Config 2's hooks on one MI355X: 7.67 ms per
        step with 256 MiB windows, 40.4 with one parameter per window, 82.9 in order on the
        caller's stream, 6.8 for the grouped step."""
        w = self._release_windows.pop(key, None)
        if w is None:
            return
        src, entries, _ = w
        gi, dev = key
        k = self._release_next % RELEASE_STREAMS
        self._release_next += 1
        st = self._chain_streams(dev, RELEASE_STREAMS)[k]
        evs = self._release_events.get(dev)
        if evs is None:
            evs = self._release_events[dev] = [torch.cuda.Event() for _ in range(RELEASE_STREAMS + 1)]
        evs[0].record(src)   # a wait takes the event as it is when enqueued, so one event serves
        st.wait_event(evs[0])
        ps = [p for p, _ in entries]
        now = [p.grad for p in ps]
        try:
            for p, g in entries:
                p.grad = g
            with torch.no_grad(), torch.cuda.stream(st):
                self._step_params(ps, _Group.from_kwargs(**self.param_groups[gi]), gi, release=True, home=src)
        finally:
            for (p, g), held in zip(entries, now):
                g.record_stream(st)   # released here, still read by the stream's step
                p.grad = held
        self._release_pending.setdefault(dev, set()).add(k)

    def _release_join(self) -> None:
        """Step what the windows still hold; then the caller's streams wait for every released
        step: for the last work of each stream that ran one (a stream runs its steps in order)."""
        for key in list(self._release_windows):
            self._release_flush(key)
        for dev, ks in self._release_pending.items():
            main = torch.cuda.current_stream(dev)
            streams = self._chain_streams(dev, RELEASE_STREAMS)
            evs = self._release_events[dev]
            for k in sorted(ks):
                evs[k + 1].record(streams[k])
                main.wait_event(evs[k + 1])
        self._release_pending = {}
        self._release_queued = False
        self._release_next = 0

    def _release_recover(self) -> None:
        """Steps and joins what a backward pass that raised left behind: its end-of-backward
        callback never ran, so its windows were not stepped and the caller's stream does not wait
        for its release streams. Called before the model's next forward, the next hook and step(),
        so the parameters are those the reference's hooks left before anything reads them.
        Nothing to do (one comparison) otherwise."""
        if self._release_queued and torch._C._current_graph_task_id() != self._release_task:
            self._release_join()

    def _release_hook_step(self, p: torch.Tensor) -> None:
        """From a post-accumulate-grad hook: the released steps of one backward pass are joined
        when it ends (a callback of the autograd engine, run on the caller's streams once they
        have waited for the gradients), before anything after backward runs."""
        self._release_recover()
        task = torch._C._current_graph_task_id()
        if not self._release_queued:
            try:
                torch.autograd.Variable._execution_engine.queue_callback(self._release_join)
                self._release_queued = True
                self._release_task = task
            except RuntimeError:   # not inside a backward pass: join at once
                pass
        self._release_step(p, join_later=self._release_queued)

    def setup_gradient_release(self, model: nn.Module, update_rate: int = 1, ignore_existing_hooks: bool = False):
        """thorn.py:1755-1776: step each parameter from its post-accumulate-grad hook (large
        orthogonalized parameters in windows on the optimizer's streams, joined when the backward
        pass ends: _release_step); the model's forward first recovers from a backward pass that
        raised (_release_recover)."""
        def _hook(param: torch.Tensor, optimizer: 'THORN'):
            optimizer._release_hook_step(cast(Parameter, param))
            param.grad = None

        def _before_forward(module: nn.Module, args, optimizer: 'THORN'):
            optimizer._release_recover()

        hooks = []
        for p in model.parameters():
            if p.requires_grad:
                if p._post_accumulate_grad_hooks is not None and len(p._post_accumulate_grad_hooks) > 0 \
                        and not ignore_existing_hooks:
                    for h in hooks:
                        if hasattr(h, 'remove'):
                            h.remove()
                    raise ValueError('Model already has post_accumulate_grad_hooks. If this is expected, '
                                     'pass `ignore_existing_hooks=True`.')
                hooks.append(p.register_post_accumulate_grad_hook(partial(_hook, optimizer=self)))
        hooks.append(model.register_forward_pre_hook(partial(_before_forward, optimizer=self)))
        model._gradient_release_hooks = hooks
        self._update_rate = update_rate
