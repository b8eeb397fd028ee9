"""Small deterministic workloads shared by the golden-vector script and the parity tests.

Each builder returns (params, groups, grad_fn): CPU fp32 leaf tensors, THORN parameter groups over
them, and grad_fn(step, index, param) giving that step's gradient (pre-drawn, so the values do not
depend on call order). Parity tests move everything to the GPU bit for bit.
"""
from __future__ import annotations

import torch


def _leaf(t: torch.Tensor) -> torch.nn.Parameter:
    return torch.nn.Parameter(t, requires_grad=True)


def _grads(gen, shapes, steps, scale, outlier_rows=0.0):
    out = {}
    for s in range(1, steps + 1):
        for i, shape in enumerate(shapes):
            g = torch.randn(shape, generator=gen) * scale
            if outlier_rows and len(shape) >= 2:
                rows = shape[-2]
                k = max(1, round(outlier_rows * rows))
                idx = torch.randperm(rows, generator=gen)[:k]
                g[..., idx, :] *= 10.0
            out[(s, i)] = g
    return out


def config1(steps: int = 10):
    """one 512x256 Linear weight, N(0, 0.02); gradients N(0, 1e-3^2), seed 3407."""
    gen = torch.Generator().manual_seed(3407)
    p = _leaf(torch.randn(512, 256, generator=gen) * 0.02)
    grads = {}
    for s in range(1, steps + 1):
        grads[(s, 0)] = torch.randn(512, 256, generator=gen) * 1e-3
    groups = [{'orthogonalize': True, 'params': [p], 'lr': 1e-3, 'betas': (0.9, 0.95), 'weight_decay': 0.1,
               'scaling_mode': 'moonlight', 'iters': 5}]
    return [p], groups, lambda s, i, prm: grads[(s, i)]


def mixed_small(steps: int = 20):
    """Tall, wide, square, batched (3-D), odd-sized and tiny matrices plus Adam tensors."""
    gen = torch.Generator().manual_seed(7)
    ortho_a = [(96, 40), (40, 96), (64, 64), (3, 24, 40), (37, 13), (32, 5)]
    ortho_b = [(33, 70), (70, 33)]
    vec = [(50,), (7,)]
    emb = [(200, 16)]
    shapes = ortho_a + ortho_b + vec + emb
    params = []
    for sh in shapes:
        init = torch.ones(sh) if len(sh) == 1 else torch.randn(sh, generator=gen) * 0.02
        params.append(_leaf(init))
    grads = _grads(gen, shapes, steps, 1e-3, outlier_rows=0.05)
    na, nb, nv = len(ortho_a), len(ortho_b), len(vec)
    groups = [
        {'orthogonalize': True, 'params': params[:na], 'lr': 2e-3, 'betas': (0.9, 0.95), 'weight_decay': 0.1},
        {'orthogonalize': True, 'params': params[na:na + nb], 'lr': 1e-3, 'betas': (0.95, 0.95),
         'weight_decay': 0.05, 'scaling_mode': 'jordan', 'force_per_neuron_norm': True},
        {'orthogonalize': False, 'params': params[na + nb:na + nb + nv], 'lr': 1e-3, 'betas': (0.9, 0.95),
         'weight_decay': 0.0, 'rectify': True},
        {'orthogonalize': False, 'params': params[na + nb + nv:], 'lr': 1e-3, 'betas': (0.9, 0.99),
         'weight_decay': 0.1, 'eps': 1e-8},
    ]
    return params, groups, lambda s, i, prm: grads[(s, i)]


def md_small(steps: int = 20):
    """decouple_md on the orthogonalized group (row/column gains and one scalar-gain group)."""
    gen = torch.Generator().manual_seed(11)
    md_split = [(48, 32), (32, 48), (40, 40), (2, 16, 24)]
    md_scalar = [(24, 36)]
    vec = [(64,)]
    shapes = md_split + md_scalar + vec
    params = []
    for sh in shapes:
        init = torch.ones(sh) if len(sh) == 1 else torch.randn(sh, generator=gen) * 0.02
        params.append(_leaf(init))
    grads = _grads(gen, shapes, steps, 1e-3, outlier_rows=0.05)
    n1, n2 = len(md_split), len(md_scalar)
    groups = [
        {'orthogonalize': True, 'params': params[:n1], 'lr': 8e-3, 'betas': (0.9, 0.95), 'weight_decay': 0.0,
         'decouple_md': True},
        {'orthogonalize': True, 'params': params[n1:n1 + n2], 'lr': 8e-3, 'betas': (0.9, 0.95),
         'weight_decay': 0.05, 'decouple_md': True, 'split_gain': False, 'scaling_mode': 'moonlight'},
        {'orthogonalize': False, 'params': params[n1 + n2:], 'lr': 1e-3, 'betas': (0.9, 0.95),
         'weight_decay': 0.0},
    ]
    return params, groups, lambda s, i, prm: grads[(s, i)]


def _with_magma(build):
    params, groups, grads = build()
    for g in groups:
        g['momentum_align'] = True
    return params, groups, grads


def magma_small(steps: int = 20):
    """mixed_small with Magma momentum-aligned masking on every group."""
    return _with_magma(lambda: mixed_small(steps))


def magma_md_small(steps: int = 20):
    """md_small with Magma momentum-aligned masking on every group (recovered direction on md)."""
    return _with_magma(lambda: md_small(steps))


def sparse_small(steps: int = 12, momentum_align: bool = False):
    """Row-sparse embedding gradients (uncoalesced, repeated rows, one empty step) beside a dense
    vector and an orthogonalized matrix."""
    gen = torch.Generator().manual_seed(23)
    shapes = [(300, 16), (64,), (64, 24)]
    params = [_leaf(torch.randn(300, 16, generator=gen) * 0.02), _leaf(torch.ones(64)),
              _leaf(torch.randn(64, 24, generator=gen) * 0.02)]
    grads = {}
    for s in range(1, steps + 1):
        nnz = 0 if s == 4 else 24
        idx = torch.randint(0, 300, (nnz,), generator=gen)
        if nnz:
            idx[-3:] = idx[:3]   # repeated rows, summed by coalesce()
        vals = torch.randn(nnz, 16, generator=gen) * 1e-3
        grads[(s, 0)] = torch.sparse_coo_tensor(idx[None], vals, (300, 16))
        grads[(s, 1)] = torch.randn(64, generator=gen) * 1e-3
        grads[(s, 2)] = torch.randn(64, 24, generator=gen) * 1e-3
    groups = [
        {'orthogonalize': False, 'params': params[:2], 'lr': 1e-3, 'betas': (0.9, 0.95), 'weight_decay': 0.1,
         'momentum_align': momentum_align},
        {'orthogonalize': True, 'params': params[2:], 'lr': 2e-3, 'betas': (0.9, 0.95), 'weight_decay': 0.1,
         'momentum_align': momentum_align},
    ]
    return params, groups, lambda s, i, prm: grads[(s, i)]


def magma_sparse_small(steps: int = 12):
    return sparse_small(steps, momentum_align=True)


def md_adam_small(steps: int = 20):
    """decouple_md on every kind of group: orthogonalized matrices with row/column gains,
    batched (3-D, 4-D) orthogonalized parameters sharing one scalar gain (split_gain=False), and
    non-orthogonalized (Adam) tensors with row/column gains, a scalar gain, rectification, and a
    per-row norm axis with the default 'init' target norm (thorn.py:594-608, 1704-1721)."""
    gen = torch.Generator().manual_seed(31)
    ortho_split = [(40, 24), (2, 12, 20)]
    ortho_scalar = [(3, 20, 28), (2, 2, 16, 12)]
    adam_split = [(60, 16), (32,), (2, 8, 12)]
    adam_scalar = [(20, 12), (16,)]
    adam_rows = [(30, 10)]
    sets = [ortho_split, ortho_scalar, adam_split, adam_scalar, adam_rows]
    shapes = [sh for st in sets for sh in st]
    params = [_leaf(torch.ones(sh) + 0.1 * torch.randn(sh, generator=gen) if len(sh) == 1
                    else torch.randn(sh, generator=gen) * 0.02) for sh in shapes]
    grads = _grads(gen, shapes, steps, 1e-3, outlier_rows=0.05)
    bounds = [0]
    for st in sets:
        bounds.append(bounds[-1] + len(st))
    ps = [params[bounds[k]:bounds[k + 1]] for k in range(len(sets))]
    groups = [
        {'orthogonalize': True, 'params': ps[0], 'lr': 8e-3, 'weight_decay': 0.0, 'decouple_md': True},
        {'orthogonalize': True, 'params': ps[1], 'lr': 4e-3, 'weight_decay': 0.05, 'decouple_md': True,
         'split_gain': False, 'gain_lr': 2e-3},
        {'orthogonalize': False, 'params': ps[2], 'lr': 2e-3, 'weight_decay': 0.1, 'decouple_md': True},
        {'orthogonalize': False, 'params': ps[3], 'lr': 2e-3, 'weight_decay': 0.0, 'decouple_md': True,
         'split_gain': False, 'rectify': True, 'eps': 1e-8, 'gain_betas': (0.8, 0.9)},
        {'orthogonalize': False, 'params': ps[4], 'lr': 1e-3, 'weight_decay': 0.1, 'decouple_md': True,
         'norm_axis': -1},
    ]
    return params, groups, lambda s, i, prm: grads[(s, i)]


def md_adam_axes(steps: int = 12):
    """decouple_md on Adam groups whose norm runs over dim -2, the columns of each trailing
    matrix (norm_axis = -2, and 0 on a 2-D tensor; thorn.py:594-595, 1717), with row/column gains
    and with a scalar gain, beside a per-row (-1) group. No golden vectors: checked against the
    oracle, whose norm is torch's over the same dims."""
    gen = torch.Generator().manual_seed(37)
    cols_split = [(48, 20), (2, 10, 14)]
    cols_scalar = [(24, 36)]
    rows = [(18, 30)]
    sets = [cols_split, cols_scalar, rows]
    shapes = [sh for st in sets for sh in st]
    params = [_leaf(torch.randn(sh, generator=gen) * 0.02) for sh in shapes]
    grads = _grads(gen, shapes, steps, 1e-3, outlier_rows=0.05)
    groups = [
        {'orthogonalize': False, 'params': params[0:2], 'lr': 2e-3, 'weight_decay': 0.1, 'decouple_md': True,
         'norm_axis': -2},
        {'orthogonalize': False, 'params': params[2:3], 'lr': 2e-3, 'weight_decay': 0.0, 'decouple_md': True,
         'split_gain': False, 'norm_axis': 0, 'eps': 1e-8},
        {'orthogonalize': False, 'params': params[3:4], 'lr': 1e-3, 'weight_decay': 0.1, 'decouple_md': True,
         'norm_axis': -1},
    ]
    return params, groups, lambda s, i, prm: grads[(s, i)]


class _MdNet(torch.nn.Module):
    def __init__(self, gen):
        super().__init__()
        self.embed = torch.nn.Embedding(40, 12)
        self.proj = torch.nn.Linear(12, 24)
        self.conv = torch.nn.Conv1d(3, 8, 5)
        self.norm = torch.nn.LayerNorm(24)
        self.lm_head = torch.nn.Linear(24, 40, bias=False)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=gen) * 0.05 + (1.0 if p.ndim == 1 else 0.0))


def md_module(steps: int = 10):
    """The nn.Module overload with decouple_md=True, as README.md:109 uses it: _auto_assign puts the
    flag into both the orthogonalized group (Linear and conv weights) and the Adam group
    (embedding, lm_head, biases, norm) (thorn.py:1302-1331). `groups` is the module and the
    constructor's keyword arguments."""
    gen = torch.Generator().manual_seed(41)
    net = _MdNet(gen)
    params = list(net.parameters())
    shapes = [tuple(p.shape) for p in params]
    grads = _grads(gen, shapes, steps, 1e-3, outlier_rows=0.05)
    return params, {'module': net, 'kwargs': {'lr': 3e-3, 'decouple_md': True}}, lambda s, i, prm: grads[(s, i)]
