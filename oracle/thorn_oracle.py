"""CPU restatement of pykeio/THORN's eager optimizer step (the parity oracle).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker or the timed CPU baseline. The product
(``thorn_amd``) never imports it and never falls back to it.

What it restates: the arithmetic that ``/root/reference/thorn/thorn.py`` runs when Triton and
``torch.compile`` are off (``THORN_DISABLE_TRITON=1``, ``THORN_COMPILE=0``, or any CPU tensor,
thorn.py:288-296, 379-385). Every function names the reference lines it follows. The in-place op
order is kept, because it fixes the fp32 rounding of the state, and Newton-Schulz runs in float16
with Gram Newton-Schulz for non-square matrices, exactly as thorn.py:626-662 does.

Left out, because they are outside the single-GPU hot path: the FSDP2/DTensor engine
(thorn.py:979-1186, 1333-1374, 1459-1581), the Triton kernels (thorn.py:53-280) and the compile
wrapper (thorn.py:379-423). Magma ``momentum_align`` (thorn.py:800-836, 1616-1634) is restated
in its single-process form.

How the pieces are pinned (tests/test_oracle.py):
  * coefficients, restarts, single-function outputs and multi-step trajectories: golden vectors
    written from the reference itself (tests/golden/make_golden.py);
  * Newton-Schulz: the f64 closed form U*phi(S)*V^T from an SVD;
  * Adam: torch.optim.Adam / RAdam special cases; per-row normalization: its invariants;
  * update_rate and gradient release: properties (the momentum and the Adam moments follow their
    recurrences every step, parameters move only on due steps, a due step is an ordinary step,
    a decouple_md parameter goes through p / G * G otherwise, hooks drop the gradients);
  * sparse (row) gradients: torch.optim.SparseAdam (eps > 0, no weight decay), untouched rows
    left alone, duplicate indices summed, an empty gradient taking no step, and reference
    trajectories with row-sparse gradients;
  * Magma: reference outputs of the PRNG and of the mask function, Magma trajectories (mixed,
    decouple_md, sparse), and properties (s stays in (0, 1], the EMA of sigmoid(cos / 2)).
"""
from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field, fields, MISSING
from functools import lru_cache
from typing import Any, Callable, Optional, Union

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.optim import Optimizer

# softplus(LN_E_SUB_1) == 1 (thorn.py:1602)
LN_E_SUB_1 = 0.5413248546


# ---------------------------------------------------------------------------------------------
# Newton-Schulz coefficients (thorn.py:425-514), host float64
# ---------------------------------------------------------------------------------------------

def _optimal_quintic(l: float, u: float) -> tuple[float, float, float]:
    """Equioscillating odd quintic on [l, u] (thorn.py:432-455)."""
    assert 0 <= l <= u
    tiny = 1e-15
    if l / u >= 1.0 - tiny:
        # degenerate interval: the classic (15/8, -10/8, 3/8) quintic scaled to u (thorn.py:436-439)
        return (15.0 / 8.0) / u, (-10.0 / 8.0) / (u ** 3.0), (3.0 / 8.0) / (u ** 5.0)
    q = (3.0 * l + u) / 4.0
    r = (l + 3.0 * u) / 4.0
    err, prev = float('inf'), None
    a = b = c = 1.0
    while not prev or abs(prev - err) > tiny:
        prev = err
        lhs = torch.tensor([
            [l, l ** 3.0, l ** 5.0, 1.0],
            [q, q ** 3.0, q ** 5.0, -1.0],
            [r, r ** 3.0, r ** 5.0, 1.0],
            [u, u ** 3.0, u ** 5.0, -1.0],
        ], dtype=torch.float64)
        a, b, c, err = torch.linalg.solve(lhs, torch.ones(4, dtype=torch.float64))
        signs = torch.tensor([-1.0, 1.0], dtype=torch.float64)
        q, r = torch.sqrt((-3.0 * b + signs * (9.0 * b ** 2.0 - 20.0 * a * c) ** 0.5) / (10.0 * c))
    return float(a), float(b), float(c)


@lru_cache(maxsize=None)
def optimal_composition(l: float, num_iters: int, safety_factor_eps: float = 0.0,
                        cushion: float = 0.0) -> list[tuple[float, float, float]]:
    """Polar-Express coefficient schedule (thorn.py:425-480)."""
    assert 0 <= l <= 1
    u = 1.0
    safety = 1.0 + safety_factor_eps
    out = []
    for it in range(num_iters):
        a, b, c = _optimal_quintic(max(l, cushion * u), u)
        if cushion * u > l:
            pl = a * l + b * l ** 3.0 + c * l ** 5.0
            pu = a * u + b * u ** 3.0 + c * u ** 5.0
            k = 2.0 / (pl + pu)
            a, b, c = a * k, b * k, c * k
        if it < num_iters - 1:
            a /= safety
            b /= safety ** 3.0
            c /= safety ** 5.0
        out.append((a, b, c))
        l = a * l + b * l ** 3.0 + c * l ** 5.0
        u = 2.0 - l
    return out


@lru_cache(maxsize=None)
def gram_ns_restarts(*coeffs: tuple[float, float, float]) -> list[int]:
    """Restart positions for Gram Newton-Schulz (thorn.py:482-514)."""
    grid = torch.logspace(0, -10, 10000, dtype=torch.float64)
    shift = -4e-4
    positions = list(range(1, len(coeffs)))
    for n_restarts in range(1, len(coeffs)):
        best, best_combo = float('inf'), []
        for combo in itertools.combinations(positions, n_restarts):
            qs = []
            e = grid.clone()
            q = r = None
            for j, (a, b, c) in enumerate(coeffs):
                if j == 0 or j in combo:
                    if j != 0:
                        e *= q
                    r = e ** 2 + shift
                    q = torch.ones(len(e), dtype=torch.float64)
                z = a + r * (b + r * c)
                q *= z
                r *= z ** 2
                qs.append(q)
            worst = max(float((t.max() / t.min()).item()) for t in qs)
            if worst < best:
                best, best_combo = worst, list(combo)
        if best < 1e8:
            return best_combo
    raise ValueError('No stable restarts with these parameters')


# ---------------------------------------------------------------------------------------------
# Parameter group (thorn.py:535-612)
# ---------------------------------------------------------------------------------------------

@dataclass
class Group:
    """Mirror of ``_THORNParameterGroup`` (thorn.py:535-612); rebuilt from the dict every step."""
    orthogonalize: bool
    params: list
    lr: float
    base_lr: float = field(init=False)
    none_grad: bool = True
    weight_decay: float = 0.1
    betas: tuple = (0.9, 0.95)
    scaling_mode: Optional[str] = None
    target_rms: float = 0.2
    target_norm: Any = None
    iters: int = 5
    rectify: bool = False
    eps: float = 0
    lower_bound: float = 1e-3
    safety_factor: float = 0.03
    cushion: float = 0.02
    momentum_align: bool = False
    coeffs: list = field(init=False)
    restarts: list = field(init=False)
    decouple_md: bool = False
    gain_lr: float = 1e-3
    gain_betas: tuple = (0.9, 0.95)
    norm_axis: Any = None
    split_gain: bool = True
    force_per_neuron_norm: bool = False

    @classmethod
    def from_dict(cls, d: dict) -> 'Group':
        return cls(**{k: d[k] for k in d if k in cls.__dataclass_fields__})

    def __post_init__(self):
        if self.lr < 0.0:
            raise ValueError(f'Invalid learning rate `{self.lr}`; should be >= 0')
        if not (0.0 <= self.betas[0] < 1.0):
            raise ValueError(f'Invalid beta1 `{self.betas[0]}`; should be in [0, 1)')
        if not (0.0 <= self.betas[1] < 1.0):
            raise ValueError(f'Invalid beta2 `{self.betas[1]}`; should be in [0, 1)')
        self.base_lr = self.lr
        self.coeffs = optimal_composition(self.lower_bound, self.iters, self.safety_factor, self.cushion)
        self.restarts = gram_ns_restarts(*self.coeffs)

    @property
    def scaling_mode_(self) -> str:
        if self.scaling_mode is None:
            return 'md' if self.decouple_md else 'moonlight'
        return self.scaling_mode

    @property
    def gain_lr_(self) -> float:
        return self.gain_lr * (float(self.lr) / self.base_lr)

    def norm_axis_(self, p):
        return self.norm_axis if self.norm_axis is not None else ((-2, -1) if p.ndim > 1 else -1)

    def target_norm_(self, p):
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


# ---------------------------------------------------------------------------------------------
# Newton-Schulz (thorn.py:298-377 eager branch, 614-667)
# ---------------------------------------------------------------------------------------------

def _dense(t):
    """GPU runs of the oracle (the large-config parity tests) hand batched products contiguous
    operands; on the CPU the operands are left exactly as the reference passes them."""
    return t.contiguous() if t.is_cuda else t


def sym_addmm(A, B, C, alpha=1.0, beta=1.0):
    """Eager branch of ``thorn::sym_addmm`` (thorn.py:321-343): beta*C + alpha*(A@B)."""
    *N, M, K = A.shape
    NN = math.prod(N)
    A = _dense(A.reshape(NN, M, K))
    B = _dense(B.reshape(NN, K, M))
    if C is not None and C.ndim != 2:
        C = C.reshape(NN, M, M)
    if C is not None:
        O = torch.baddbmm(C, A, B, alpha=float(alpha), beta=float(beta))
    else:
        O = torch.bmm(A, B).mul_(float(alpha))
    return O.reshape(*N, M, M)


def baddbmm_nd(inp, b1, b2, alpha=1.0, beta=1.0):
    """thorn.py:614-624: baddbmm over arbitrary leading dims."""
    *N, M, K = b1.shape
    P = b2.shape[-1]
    NN = math.prod(N)
    return torch.baddbmm(inp.broadcast_to((*N, M, P)).reshape(NN, M, P), _dense(b1.reshape(NN, M, K)),
                         _dense(b2.reshape(NN, K, P)), alpha=alpha, beta=beta).reshape(*N, M, P)


def polar_decomp(X: torch.Tensor, coeffs, restarts) -> torch.Tensor:
    """Float16 Newton-Schulz polar factor (thorn.py:626-662).

    Square matrices run the plain quintic; non-square ones run Gram Newton-Schulz on X X^T with
    the given restarts. Tall inputs are transposed first and back at the end.
    """
    dtype = X.dtype
    gram = max(X.shape[-2:]) > min(X.shape[-2:])
    transposed = X.size(-2) > X.size(-1)
    if transposed:
        X = X.mT
    X = X.to(torch.float32)
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + 1e-8)
    X = X.to(torch.float16)
    if gram:
        eye = torch.eye(X.size(-2), device=X.device, dtype=X.dtype)
        R = sym_addmm(X, X.mT, None)
        Q = None
        for i, (a, b, c) in enumerate(coeffs):
            if i in restarts and i != 0:
                X = _dense(Q) @ _dense(X)
                R = sym_addmm(X, X.mT, None)
            Z = sym_addmm(R, R, R, alpha=c, beta=b)
            Q = sym_addmm(Q, Z, Q, beta=a) if i != 0 and i not in restarts else Z + a * eye
            if i < len(coeffs) - 1 and i + 1 not in restarts:
                RZ = sym_addmm(R, Z, R, beta=a)
                R = sym_addmm(Z, RZ, RZ, beta=a)
        X = _dense(X.mT) @ _dense(Q) if transposed else _dense(Q) @ _dense(X)
    else:
        for (a, b, c) in coeffs:
            A = sym_addmm(X, X.mT, None)
            B = sym_addmm(A, A, A, alpha=c, beta=b)
            X = baddbmm_nd(X, B, X, beta=a)
        X = X.mT if transposed else X
    return X.to(dtype=dtype)


def polar_closed_form(X: torch.Tensor, coeffs) -> torch.Tensor:
    """f64 closed form of the same map: U * phi(S) * V^T, phi = p_k o ... o p_1 (no rounding).

    Both the plain quintic and Gram Newton-Schulz equal this in exact arithmetic, after the
    Frobenius normalization of thorn.py:633.
    """
    Xd = X.to(torch.float64)
    Xd = Xd / (Xd.norm(dim=(-2, -1), keepdim=True) + 1e-8)
    U, S, Vh = torch.linalg.svd(Xd, full_matrices=False)
    for a, b, c in coeffs:
        S = a * S + b * S ** 3 + c * S ** 5
    return (U * S.unsqueeze(-2)) @ Vh


# ---------------------------------------------------------------------------------------------
# Update math (thorn.py:669-798, 838-888)
# ---------------------------------------------------------------------------------------------

def cautious_weight_decay(p, update, wd):
    """Cautious weight decay (thorn.py:669-681): u += wd * p where u * p >= 0."""
    if wd > 0.0:
        mask = ((update * p) >= 0).to(dtype=p.dtype)
        update.addcmul_(p, mask.mul_(wd))
    return update


def weight_decay_update(p, update, *, weight_decay: float, lr: float):
    """thorn.py:683-702 (eager branch :702)."""
    p.data.sub_(cautious_weight_decay(p, update, weight_decay), alpha=lr)


def needs_neuron_norm(p, group: Group) -> bool:
    """thorn.py:704-707: tall matrices only, unless forced; beta2 == 0 switches it off."""
    return group.betas[1] > 0 and (p.size(-2) > p.size(-1) or group.force_per_neuron_norm)


def per_neuron_norm_update(p, u, *, lr=0.0, weight_decay=0.0):
    """Stateless per-row normalization (thorn.py:709-766, eager branch :758-766)."""
    eps = float(torch.finfo(u.dtype).eps)
    v_norm = u.norm(dim=(-2, -1), keepdim=True)
    v_mean = u.square().mean(dim=-1, keepdim=True)
    u.mul_(v_mean.clamp_min(eps).rsqrt_())
    v_norm_new = u.norm(dim=(-2, -1), keepdim=True)
    u.mul_(v_norm.div(v_norm_new.clamp_min(eps)))
    if p is not None:
        weight_decay_update(p, u, weight_decay=weight_decay, lr=lr)
    return u


def lr_scale_ortho(p, group: Group) -> float:
    """thorn.py:768-780."""
    mode = group.scaling_mode_
    if mode == 'md':
        d_out, d_in = p.size(-2), p.size(-1)
        return max(d_out / d_in, d_in / d_out) ** 0.5
    if mode == 'moonlight':
        assert group.target_rms > 0
        return group.target_rms * (max(1, *p.shape[-2:]) ** 0.5)
    if mode == 'jordan':
        return max(1, p.size(-2) / p.size(-1)) ** 0.5
    raise ValueError(mode)


def compute_rect(group: Group, step) -> float:
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


def w1rand(s: int) -> tuple[int, int]:
    """64-bit hash PRNG of Magma masking (thorn.py:800-804): a Weyl step s += C, then the xor of the
    two halves of the 128-bit product s * (s ^ C)."""
    C = 0xD07EBC63274654C7
    s = (s + C) & 0xFFFFFFFFFFFFFFFF
    t = s * (s ^ C)
    return s, ((t >> 64) ^ t) & 0xFFFFFFFFFFFFFFFF


def momentum_aligned_mask(g, state, group: Group, *, tau=2.0, p=0.9, moment=None) -> float:
    """Magma masking, single-process branch (thorn.py:806-836): s <- p s + (1 - p) sigmoid(cos(g, m)
    / tau) with the moment before this step's update; the step is skipped (0.0) when the PRNG
    draw is odd, otherwise the learning rate is scaled by s."""
    if not group.momentum_align:
        return 1.0
    g_flat = g.flatten()
    m_flat = (state['moment'] if moment is None else moment).flatten()
    s_t = torch.sigmoid(nn.functional.cosine_similarity(g_flat, m_flat, dim=0) / tau)
    state['s'] = p * state['s'] + (1 - p) * s_t
    state['random_state'], mask = w1rand(state['random_state'])
    if mask % 2 != 0:
        return 0.0
    return state['s'].item()


def adam_update(p, g, momentum, variance, step, *, beta1, beta2, lr, weight_decay, eps,
                degenerate=False):
    """Adam / Adam-atan2 with cautious weight decay (thorn.py:838-888, eager branch :876-888)."""
    bc1 = 1 / (1 - beta1 ** step)
    bc2 = 1 / (1 - beta2 ** step)
    momentum.lerp_(g, weight=1 - beta1)
    variance.mul_(beta2).addcmul_(g, g, value=1 - beta2)
    if not degenerate:
        if eps == 0.0:
            u = torch.atan2(momentum * bc1, (variance * bc2).sqrt_())
        else:
            u = (momentum * bc1) / (variance * bc2).sqrt_().add_(eps)
    else:
        u = momentum.clone()
    if p is not None:
        weight_decay_update(p, u, weight_decay=weight_decay, lr=lr)


# ---------------------------------------------------------------------------------------------
# Decoupled magnitude / direction (thorn.py:890-977)
# ---------------------------------------------------------------------------------------------

def recover_direction(p, state):
    """thorn.py:890-908: p /= gain; p_g = p * g; g *= gain (in place)."""
    g = p.grad
    assert g is not None
    if 'row_gain' in state:
        row_gain = F.softplus(state['row_gain'])
        col_gain = F.softplus(state['col_gain'])
        gain, gains = row_gain * col_gain, (row_gain, col_gain)
    else:
        gain = F.softplus(state['gain'])
        gains = None
    p.div_(gain)
    p_g = p * g
    g.mul_(gain)
    return g, p_g, gains


def update_magnitude(p_g, gain, gain2, dim, moment, variance, state, group: Group):
    """thorn.py:910-932: Adam-atan2 step on a gain vector from sum(p*g*other_gain)*sigmoid(gain)."""
    d_gain = torch.sigmoid(gain)
    if gain2 is not None:
        p_g = p_g * gain2
    grad = p_g.sum(dim=dim).mul_(d_gain.squeeze(dim) if dim is not None else d_gain)
    adam_update(gain, grad.unsqueeze(dim) if dim is not None else grad, moment, variance,
                state['step'], beta1=group.gain_betas[0], beta2=group.gain_betas[1],
                lr=group.gain_lr_, weight_decay=0.0, eps=group.eps)


def update_magnitudes(p_g, gains, state, group: Group):
    """thorn.py:934-967: row gain first, then column gain with the *old* row softplus."""
    if 'row_gain' in state:
        assert gains is not None
        update_magnitude(p_g, state['row_gain'], gains[1], -1, state['row_gain_moment'],
                         state['row_gain_variance'], state, group)
        update_magnitude(p_g, state['col_gain'], gains[0], -2, state['col_gain_moment'],
                         state['col_gain_variance'], state, group)
    else:
        update_magnitude(p_g, state['gain'], None, None, state['gain_moment'],
                         state['gain_variance'], state, group)


def reassemble_md(p, state):
    """thorn.py:969-977: p *= softplus(row_gain); p *= softplus(col_gain) (or the scalar gain)."""
    if 'row_gain' in state:
        p.mul_(F.softplus(state['row_gain']))
        p.mul_(F.softplus(state['col_gain']))
    else:
        p.mul_(F.softplus(state['gain']))


# ---------------------------------------------------------------------------------------------
# Optimizer (thorn.py:1229-1331, 1376-1457, 1583-1753), single process, dense gradients
# ---------------------------------------------------------------------------------------------

_GROUP_DEFAULTS = {}
for _f in fields(Group):
    if _f.default is not MISSING:
        _GROUP_DEFAULTS[_f.name] = _f.default
    elif _f.default_factory is not MISSING:  # pragma: no cover - no factories above
        _GROUP_DEFAULTS[_f.name] = _f.default_factory()


class OracleTHORN(Optimizer):
    """CPU restatement of ``THORN`` (thorn.py:1229): same groups, state keys and step order."""

    polar_decomp_batch_size: int = 32 * 1024 * 1024

    def __init__(self, params, **conf):
        self._update_rate = 1
        groups = auto_assign(params, **conf) if isinstance(params, nn.Module) else params
        for g in groups:
            assert 'orthogonalize' in g
            if g['orthogonalize']:
                assert all(p.ndim >= 2 for p in g['params']), \
                    'Only parameters with ndim >= 2 can be orthogonalized'
        super().__init__(groups, dict(_GROUP_DEFAULTS))
        self._param_to_group = {id(p): g for g in self.param_groups for p in g['params']}

    # thorn.py:1376-1381
    def _update_momentum(self, p, g, group: Group):
        m = self.state[p]['moment']
        m.mul_(group.betas[0]).add_(g)
        return g.add(m, alpha=group.betas[0])

    # thorn.py:1383-1397
    def _ortho_pre(self, p, group: Group):
        state = self.state[p]
        g = p.grad
        p_g = gains = None
        if group.decouple_md:
            g, p_g, gains = recover_direction(p, state)
        magma = momentum_aligned_mask(g, state, group)
        u = self._update_momentum(p, g, group)
        if magma == 0.0 or (state['step'] + 1) % self._update_rate != 0:
            u = None
        return u, (g, p_g, gains, magma)

    # thorn.py:1399-1425
    def _ortho_post(self, p, group: Group, u, ctx):
        g, p_g, gains, magma = ctx
        state = self.state[p]
        if u is not None:
            u = u.to(dtype=p.dtype)
            lr = group.lr * lr_scale_ortho(u, group) * magma
            if needs_neuron_norm(p, group):
                per_neuron_norm_update(p, u, lr=lr, weight_decay=group.weight_decay)
            else:
                weight_decay_update(p, u, weight_decay=group.weight_decay, lr=lr)
            if group.decouple_md:
                p.mul_(state['target_norm'] / (p.norm(dim=(-2, -1), keepdim=True) + 1e-8))
                update_magnitudes(p_g, gains, state, group)
        if group.decouple_md:
            reassemble_md(p, state)
        if group.none_grad:
            p.grad = None

    # thorn.py:1427-1457
    def _batched_ortho_step(self, params, group: Group):
        pending = []
        buckets: dict = {}
        for p in params:
            u, ctx = self._ortho_pre(p, group)
            if u is not None:
                pending.append([p, u, ctx])
                buckets.setdefault((tuple(u.shape), u.dtype, u.device), []).append(len(pending) - 1)
            else:
                self._ortho_post(p, group, None, ctx)
        coeffs, restarts = tuple(group.coeffs[:group.iters]), tuple(group.restarts)
        for (shape, _, _), idxs in buckets.items():
            bs = max(1, self.polar_decomp_batch_size // max(1, math.prod(shape)))
            for s in range(0, len(idxs), bs):
                batch = idxs[s:s + bs]
                if len(batch) == 1:
                    outs = (polar_decomp(pending[batch[0]][1], coeffs, restarts),)
                else:
                    u = torch.stack([pending[i][1] for i in batch])
                    for i in batch:
                        pending[i][1] = None
                    outs = polar_decomp(u, coeffs, restarts).unbind(0)
                    del u
                for i, u in zip(batch, outs):
                    p, _, ctx = pending[i]
                    self._ortho_post(p, group, u, ctx)

    # thorn.py:1583-1732 (no DTensor)
    def _step_params(self, params, group: Group):
        regular = []
        for p in params:
            g = p.grad
            if p is None or g is None:
                continue
            state = self.state[p]
            if 'step' not in state:
                state['step'] = 1
                state['moment'] = torch.zeros_like(p)
                if not group.orthogonalize:
                    state['variance'] = torch.zeros_like(p)
                if group.decouple_md:
                    if p.ndim > 1 and group.split_gain:
                        state['row_gain'] = torch.full((*p.shape[:-1], 1), LN_E_SUB_1, dtype=p.dtype, device=p.device)
                        state['col_gain'] = torch.full((*p.shape[:-2], 1, *p.shape[-1:]), LN_E_SUB_1, dtype=p.dtype, device=p.device)
                        for k in ['row_gain', 'col_gain']:
                            state[f'{k}_moment'] = torch.zeros_like(state[k])
                            state[f'{k}_variance'] = torch.zeros_like(state[k])
                    else:
                        state['gain'] = torch.full((), LN_E_SUB_1, dtype=p.dtype, device=p.device)
                        state['gain_moment'] = torch.zeros((), dtype=p.dtype, device=p.device)
                        state['gain_variance'] = torch.zeros((), dtype=p.dtype, device=p.device)
                    state['target_norm'] = group.target_norm_(p)
                if group.momentum_align:
                    # thorn.py:1616-1621: drawn from the generator of the gradient's device
                    state['random_state'] = torch.randint(0, (1 << 63) - 1, (), device=p.grad.device,
                                                          dtype=torch.uint64).item()
                    state['s'] = torch.ones((), dtype=p.dtype, device=p.device)
            regular.append(p)

        batched = []
        for p in regular:
            state = self.state[p]
            if group.orthogonalize:
                batched.append(p)
                continue
            g = p.grad
            step = state['step']
            beta1, beta2 = group.betas
            rect = compute_rect(group, step)
            # thorn.py:1667-1700: a row-sparse gradient updates only its rows (lazy Adam)
            if g.is_sparse and (group.decouple_md or g.sparse_dim() != 1):
                p.grad = g = g.to_dense()
            elif g.is_sparse:
                g = g.coalesce()
                g_rows = g.values()
                idxs = g.indices()[0]
                if idxs.numel() == 0:
                    continue
                moment_rows = state['moment'].index_select(0, idxs)
                variance_rows = state['variance'].index_select(0, idxs)
                magma = momentum_aligned_mask(g_rows, state, group, moment=moment_rows)
                apply = magma != 0.0 and (step + 1) % self._update_rate == 0
                p_rows = p.index_select(0, idxs) if apply else None
                adam_update(p_rows, g_rows, moment_rows, variance_rows, step, beta1=beta1, beta2=beta2,
                            lr=group.lr * rect * magma, weight_decay=group.weight_decay, eps=group.eps,
                            degenerate=rect == 0.0)
                state['moment'].index_copy_(0, idxs, moment_rows)
                state['variance'].index_copy_(0, idxs, variance_rows)
                if p_rows is not None:
                    p.index_copy_(0, idxs, p_rows)
                state['step'] += 1
                if group.none_grad:
                    p.grad = None
                continue
            magma = momentum_aligned_mask(g, state, group)
            if group.decouple_md:
                g, p_g, gains = recover_direction(p, state)
            apply = magma != 0.0 and (step + 1) % self._update_rate == 0
            adam_update(p if apply else None, g, state['moment'], state['variance'], state['step'],
                        beta1=beta1, beta2=beta2, lr=group.lr * rect * magma,
                        weight_decay=group.weight_decay, eps=group.eps, degenerate=rect == 0.0)
            if apply and group.decouple_md:
                p.mul_(state['target_norm'] / (p.norm(dim=group.norm_axis_(p), keepdim=True) + 1e-8))
                update_magnitudes(p_g, gains, state, group)
            if group.decouple_md:
                reassemble_md(p, state)
            if group.none_grad:
                p.grad = None
            state['step'] += 1

        if batched:
            self._batched_ortho_step(batched, group)
            for p in batched:
                self.state[p]['step'] += 1

    # thorn.py:1734-1753
    @torch.no_grad()
    def step(self, closure: Optional[Callable[[], float]] = None, *, param=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if param is None:
            for group in self.param_groups:
                self._step_params(group['params'], Group.from_dict(group))
        else:
            self._step_params([param], Group.from_dict(self._param_to_group[id(param)]))
        return loss


    # thorn.py:1755-1776
    def setup_gradient_release(self, model: nn.Module, update_rate: int = 1, ignore_existing_hooks: bool = False):
        """Every parameter steps from its post-accumulate-grad hook (step(param=p), then its grad is
        dropped); update_rate > 1 makes only every update_rate-th step of a parameter update it."""
        def hook(param, optimizer):
            optimizer.step(param=param)
            param.grad = None

        hooks = []
        for prm in model.parameters():
            if not prm.requires_grad:
                continue
            if prm._post_accumulate_grad_hooks and not ignore_existing_hooks:
                for h in hooks:
                    h.remove()
                raise ValueError('Model already has post_accumulate_grad_hooks. If this is expected, '
                                 'pass `ignore_existing_hooks=True`.')
            hooks.append(prm.register_post_accumulate_grad_hook(lambda t, o=self: hook(t, o)))
        model._gradient_release_hooks = hooks
        self._update_rate = update_rate


def auto_assign(module: nn.Module, **keys) -> list[dict]:
    """thorn.py:1302-1331: ndim>=2, not 'lm_head', not an nn.Embedding weight -> orthogonalized."""
    emb = set()
    module.apply(lambda m: emb.add(id(m.weight)) if isinstance(m, nn.Embedding) else None)
    ortho, regular = [], []
    for name, prm in module.named_parameters():
        if prm.ndim >= 2 and 'lm_head' not in name and id(prm) not in emb:
            ortho.append(prm)
        else:
            regular.append(prm)
    return [{'orthogonalize': True, 'params': ortho, **keys},
            {'orthogonalize': False, 'params': regular, **keys}]
