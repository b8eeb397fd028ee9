"""Writes golden vectors from the reference implementation itself (run in the build container only).

The reference (/root/reference/thorn/thorn.py, pykeio/THORN 3.1.1) targets Python >= 3.12. Two
lines keep it from importing on this image's Python 3.10, and neither touches arithmetic:
  * ``typing.NotRequired`` (3.11+) is taken from ``typing_extensions`` instead;
  * ``_optional_compile`` uses PEP 695 syntax (``def f[T: Callable](fn: T) -> T``); the type
    parameter becomes a module-level ``TypeVar`` (the body only passes it to ``typing.cast``).
    With THORN_COMPILE=0 that wrapper returns the eager function anyway (thorn.py:394-405).
The module is executed from that text in memory (nothing from the reference is written to disk)
with THORN_DISABLE_TRITON=1 and THORN_COMPILE=0, on CPU tensors, with one thread. The outputs are
small .npz fixtures next to this script; only they are committed.

What the fixtures pin, and why they need the reference itself (closed forms cover the rest):
  * coeffs_*.npz      - _optimal_composition and _gram_ns_restarts at several settings;
  * polar_*.npz       - _polar_decomp_impl: the reference's float16 Gram/plain NS trajectory;
  * pnn.npz, adam.npz - single-function outputs of _per_neuron_norm_update and _adam_update;
  * traj_config1.npz  - 10 full THORN steps on the 512x256 Linear of BASELINE config 1;
  * traj_mixed.npz    - 20 steps over a mixed set (tall/wide/square/3-D/vectors, rectify, eps>0);
  * traj_md.npz       - 20 steps with decouple_md on the orthogonalized group (config-3 branch);
  * magma.npz         - _w1rand sequences and _momentum_aligned_mask outputs (Magma);
  * traj_magma*.npz   - Magma trajectories: the mixed and decouple_md sets with momentum_align on
    every group, and row-sparse embedding gradients with and without it;
  * traj_md_adam.npz  - 20 steps with decouple_md on orthogonalized and Adam groups (row/column
    gains, scalar gains shared by batched matrices, rectification, a per-row norm axis);
  * traj_md_module.npz - 10 steps of THORN(module, decouple_md=True) (the nn.Module overload).

Usage: python tests/golden/make_golden.py [fixture ...]   (e.g. `magma traj_magma`; default: all)
"""
from __future__ import annotations

import os
import re
import sys
import types
from pathlib import Path

import numpy as np

os.environ['THORN_DISABLE_TRITON'] = '1'
os.environ['THORN_COMPILE'] = '0'

import torch  # noqa: E402

HERE = Path(__file__).resolve().parent
REF = Path('/root/reference/thorn/thorn.py')
sys.path.insert(0, str(HERE.parent.parent))
from tests.golden import workloads  # noqa: E402


def load_reference() -> types.ModuleType:
    src = REF.read_text()
    src, n1 = re.subn(r'from typing import ([^\n]*?), NotRequired, ',
                      r'from typing_extensions import NotRequired\nfrom typing import \1, ', src, count=1)
    src, n2 = re.subn(r'def _optional_compile\[T: Callable\]\(fn: T\) -> T:',
                      "T = __import__('typing').TypeVar('T')\ndef _optional_compile(fn):", src, count=1)
    if (n1, n2) != (1, 1):
        raise RuntimeError('reference source changed; compatibility edits did not apply')
    mod = types.ModuleType('thorn_reference')
    mod.__file__ = str(REF)
    sys.modules['thorn_reference'] = mod
    exec(compile(src, str(REF), 'exec'), mod.__dict__)
    assert not mod._use_triton
    return mod


def save(name: str, **arrays) -> None:
    out = {k: (v.detach().cpu().numpy() if torch.is_tensor(v) else np.asarray(v)) for k, v in arrays.items()}
    np.savez_compressed(HERE / name, **out)
    print(f'wrote {name}: {sum(a.nbytes for a in out.values()) / 1024:.0f} KiB raw')


def coefficient_fixtures(ref) -> None:
    settings = [(1e-3, 5, 0.03, 0.02), (1e-3, 8, 0.03, 0.02), (1e-2, 5, 0.0, 0.0), (1e-3, 5, 0.01, 0.0),
                (0.5, 3, 0.03, 0.02)]
    coeffs, restarts, lens = [], [], []
    for l, it, sf, cu in settings:
        c = ref._optimal_composition(l=l, num_iters=it, safety_factor_eps=sf, cushion=cu)
        r = ref._gram_ns_restarts(*c)
        coeffs.append(np.asarray(c, dtype=np.float64).reshape(-1, 3))
        restarts.append(np.asarray(r + [-1] * (8 - len(r)), dtype=np.int64))
        lens.append(it)
    save('coeffs.npz', settings=np.asarray(settings, dtype=np.float64),
         coeffs=np.concatenate(coeffs), iters=np.asarray(lens), restarts=np.stack(restarts))


def polar_fixtures(ref) -> None:
    g = torch.Generator().manual_seed(1234)
    coeffs = tuple(ref._optimal_composition(l=1e-3, num_iters=5, safety_factor_eps=0.03, cushion=0.02))
    restarts = tuple(ref._gram_ns_restarts(*coeffs))
    out = {}
    for k, shape in enumerate([(32, 32), (24, 56), (56, 24), (3, 16, 40), (5, 3), (64, 192), (128, 64)]):
        x = torch.randn(shape, generator=g) * 1e-2
        y = ref._polar_decomp_impl(x, coeffs, restarts)
        out[f'in{k}'] = x
        out[f'out{k}'] = y
    save('polar.npz', **out)


def pnn_adam_fixtures(ref) -> None:
    g = torch.Generator().manual_seed(99)
    u = torch.randn(96, 40, generator=g)
    u[::7] *= 30.0
    p = torch.randn(96, 40, generator=g) * 0.02
    p0, u0 = p.clone(), u.clone()
    ref._per_neuron_norm_update(p, u, lr=3e-3, weight_decay=0.1)
    save('pnn.npz', u_in=u0, p_in=p0, u_out=u, p_out=p)

    out = {}
    cases = [dict(eps=0.0, weight_decay=0.1, degenerate=False), dict(eps=1e-8, weight_decay=0.0, degenerate=False),
             dict(eps=0.0, weight_decay=0.05, degenerate=True)]
    for k, case in enumerate(cases):
        p = torch.randn(1000, generator=g) * 0.02
        m = torch.randn(1000, generator=g) * 1e-3
        v = torch.rand(1000, generator=g) * 1e-6
        out[f'p{k}'], out[f'm{k}'], out[f'v{k}'] = p.clone(), m.clone(), v.clone()
        for step in (1, 2, 7):
            gr = torch.randn(1000, generator=g) * 1e-3
            out[f'g{k}_{step}'] = gr.clone()
            ref._adam_update(p, gr, m, v, step, beta1=0.9, beta2=0.95, lr=1e-3, **case)
            out[f'p{k}_{step}'], out[f'm{k}_{step}'], out[f'v{k}_{step}'] = p.clone(), m.clone(), v.clone()
    save('adam.npz', **out)


def magma_fixtures(ref) -> None:
    out = {}
    seeds = [0, 1, 2, 0xD07EBC63274654C7, (1 << 63) - 2, (1 << 64) - 1, 0x0123456789ABCDEF, 987654321987654321]
    states, draws = [], []
    for seed in seeds:
        st, row_s, row_d = seed, [], []
        for _ in range(40):
            st, d = ref._w1rand(st)
            row_s.append(st)
            row_d.append(d)
        states.append(row_s)
        draws.append(row_d)
    out['w1_seeds'] = np.asarray(seeds, dtype=np.uint64)
    out['w1_states'] = np.asarray(states, dtype=np.uint64)
    out['w1_draws'] = np.asarray(draws, dtype=np.uint64)

    g = torch.Generator().manual_seed(4321)
    group = types.SimpleNamespace(momentum_align=True)
    k = 0
    for shape, mode, s0 in [((64,), 'zero', 1.0), ((64,), 'aligned', 0.8), ((64,), 'opposed', 0.6),
                            ((24, 40), 'aligned', 0.9), ((3, 8, 12), 'random', 0.5),
                            ((5, 16), 'rows', 0.7), ((1000,), 'random', 0.95), ((16, 16), 'tiny', 0.3)]:
        gr = torch.randn(shape, generator=g) * 1e-3
        noise = torch.randn(shape, generator=g) * 1e-3
        m = {'zero': torch.zeros(shape), 'aligned': 0.7 * gr + 0.3 * noise, 'opposed': -0.5 * gr + 0.2 * noise,
             'random': noise, 'rows': noise, 'tiny': gr * 1e-30}[mode]
        for seed in (seeds[k % len(seeds)], seeds[(k + 3) % len(seeds)]):
            state = {'s': torch.tensor(s0), 'random_state': seed}
            if mode == 'rows':   # the sparse path passes the gathered moment rows (thorn.py:1679)
                state['moment'] = torch.full(shape, 123.0)
                scale = ref._momentum_aligned_mask(gr, state, group, moment=m)
            else:
                state['moment'] = m
                scale = ref._momentum_aligned_mask(gr, state, group)
            out[f'mask{k}_g'], out[f'mask{k}_m'] = gr, m
            out[f'mask{k}_s0'] = np.float32(s0)
            out[f'mask{k}_seed'] = np.uint64(seed)
            out[f'mask{k}_rows'] = np.bool_(mode == 'rows')
            out[f'mask{k}_scale'] = np.float64(scale)
            out[f'mask{k}_s1'] = state['s']
            out[f'mask{k}_state1'] = np.uint64(state['random_state'])
            k += 1
    out['n_mask'] = np.int64(k)
    save('magma.npz', **out)


def run_trajectory(ref, name: str, build, steps: int, snapshot_every: int) -> None:
    torch.manual_seed(0)
    params, groups, grads = build()
    if isinstance(groups, dict):   # the nn.Module overload
        opt = ref.THORN(groups['module'], **groups['kwargs'])
    else:
        opt = ref.THORN(groups)
    out = {}
    for i, p in enumerate(params):
        out[f'init_p{i}'] = p.detach().clone()
    for s in range(1, steps + 1):
        for i, p in enumerate(params):
            p.grad = grads(s, i, p).clone()
        opt.step()
        if s % snapshot_every == 0 or s == 1:
            for i, p in enumerate(params):
                out[f's{s}_p{i}'] = p.detach().clone()
                for k, v in opt.state[p].items():
                    if torch.is_tensor(v):
                        out[f's{s}_{k}{i}'] = v.clone()
                    else:
                        out[f's{s}_{k}{i}'] = np.asarray(v)
    save(name, **out)


def main(only: list[str]) -> None:
    """Writes every fixture, or only those whose file names start with one of `only`."""
    torch.set_num_threads(1)
    ref = load_reference()
    jobs = [
        ('coeffs', lambda: coefficient_fixtures(ref)),
        ('polar', lambda: polar_fixtures(ref)),
        ('pnn', lambda: pnn_adam_fixtures(ref)),
        ('traj_config1', lambda: run_trajectory(ref, 'traj_config1.npz', workloads.config1, 10, 10)),
        ('traj_mixed', lambda: run_trajectory(ref, 'traj_mixed.npz', workloads.mixed_small, 20, 10)),
        ('traj_md', lambda: run_trajectory(ref, 'traj_md.npz', workloads.md_small, 20, 10)),
        ('magma', lambda: magma_fixtures(ref)),
        ('traj_magma', lambda: run_trajectory(ref, 'traj_magma.npz', workloads.magma_small, 20, 10)),
        ('traj_magma_md', lambda: run_trajectory(ref, 'traj_magma_md.npz', workloads.magma_md_small, 20, 10)),
        ('traj_sparse', lambda: run_trajectory(ref, 'traj_sparse.npz', workloads.sparse_small, 12, 4)),
        ('traj_magma_sparse', lambda: run_trajectory(ref, 'traj_magma_sparse.npz', workloads.magma_sparse_small,
                                                     12, 4)),
        ('traj_md_adam', lambda: run_trajectory(ref, 'traj_md_adam.npz', workloads.md_adam_small, 20, 10)),
        ('traj_md_module', lambda: run_trajectory(ref, 'traj_md_module.npz', workloads.md_module, 10, 5)),
    ]
    for name, job in jobs:
        if not only or name in only:
            job()


if __name__ == '__main__':
    main(sys.argv[1:])
