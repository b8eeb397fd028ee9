"""thorn_ortho_step_noalloc (the allocation-free variant of thorn_ortho_fill_table + thorn_ortho_step,
its workspace in the library's static device array) against the existing entry point on a fresh
caller workspace: two calls in a row, the second with a smaller matrix set on the array the first
left dirty; results bit-identical (same kernels, same exact first iterate). Plans too large for
the array are refused before anything runs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = 'cuda:0'


def _setup(shapes, seed):
    from thorn_amd import _coeffs, _lib
    gen = torch.Generator(device=DEV).manual_seed(seed)
    rows = [r for r, _ in shapes]
    cols = [c for _, c in shapes]
    flags = [_lib.MAT_PER_ROW_NORM if r > c else 0 for r, c in shapes]
    p = [torch.randn(sh, generator=gen, device=DEV) * 0.02 for sh in shapes]
    g = [torch.randn(sh, generator=gen, device=DEV) * 1e-3 for sh in shapes]
    m = [torch.randn(sh, generator=gen, device=DEV) * 1e-3 for sh in shapes]
    c = _coeffs.ns_coefficients(1e-3, 5, 0.03, 0.02)
    coeffs = np.asarray(c, dtype=np.float32).reshape(-1, 3)
    mask = sum(1 << i for i in _coeffs.gram_restarts(c) if 0 < i < 5)
    return rows, cols, flags, p, g, m, coeffs, mask


def _steps(lib, p, g, m, shapes):
    steps = np.zeros(len(p), dtype=lib.ORTHO_MAT_STEP)
    for i, (pp, gg, mm) in enumerate(zip(p, g, m)):
        steps[i]['p'], steps[i]['g'], steps[i]['m'] = pp.data_ptr(), gg.data_ptr(), mm.data_ptr()
        r, c = shapes[i]
        steps[i]['eta'] = 1e-2 * 0.2 * max(r, c) ** 0.5
        steps[i]['weight_decay'] = 0.1
        steps[i]['beta1'] = 0.9
        steps[i]['step_flags'] = lib.STEP_APPLY
    return steps


def _compare(shapes, seed):
    from thorn_amd import _lib
    rows, cols, flags, p, g, m, coeffs, mask = _setup(shapes, seed)
    stream = torch.cuda.current_stream().cuda_stream
    # existing entry points on a caller-allocated workspace
    pa, ga, ma = [t.clone() for t in p], [t.clone() for t in g], [t.clone() for t in m]
    plan_a = _lib.OrthoPlan(rows, cols, flags)
    ws = torch.zeros(plan_a.workspace_bytes, dtype=torch.uint8, device=DEV)
    table = torch.empty(max(64, plan_a.table_bytes), dtype=torch.uint8, device=DEV)
    host = torch.empty(plan_a.table_bytes, dtype=torch.uint8, pin_memory=True)
    plan_a.fill_table(_steps(_lib, pa, ga, ma, shapes), ws.data_ptr(), table.data_ptr(), host.data_ptr())
    table[:plan_a.table_bytes].copy_(host, non_blocking=True)
    plan_a.step(table.data_ptr(), coeffs, mask, stream)
    # the no-alloc entry point on copies of the same inputs
    pb, gb, mb = [t.clone() for t in p], [t.clone() for t in g], [t.clone() for t in m]
    plan_b = _lib.OrthoPlan(rows, cols, flags)
    plan_b.step_noalloc(_steps(_lib, pb, gb, mb, shapes), coeffs, mask, stream)
    torch.cuda.synchronize()
    for i, sh in enumerate(shapes):
        assert not torch.equal(pa[i], p[i]), (sh, 'the step moved nothing')
        assert torch.equal(pa[i], pb[i]), (sh, (pa[i] - pb[i]).abs().max().item())
        assert torch.equal(ma[i], mb[i]), sh
    print(f'[gpu] no-alloc step matches the existing entry point bit for bit on {shapes}', flush=True)


def test_noalloc_matches_existing_entry_point_twice():
    # large (grouped 256 x 256 path, per-row normalized), square, and small (one-launch path)
    # matrices, then a smaller set on the array the first call left dirty
    _compare([(2048, 1024), (512, 512), (96, 200), (40, 24)], seed=5)
    _compare([(300, 7)], seed=6)


def test_noalloc_refuses_plans_beyond_the_array():
    from thorn_amd import _lib
    plan = _lib.OrthoPlan([4096], [4096], [0])   # 32 MiB of iterates alone
    assert plan.workspace_bytes > _lib.NOALLOC_SCRATCH_BYTES
    steps = np.zeros(1, dtype=_lib.ORTHO_MAT_STEP)
    coeffs = np.zeros((5, 3), dtype=np.float32)
    with pytest.raises(_lib.ThornError, match='no-alloc limit'):
        plan.step_noalloc(steps, coeffs, 0, torch.cuda.current_stream().cuda_stream)
