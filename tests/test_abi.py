"""The C ABI library loads, exports every symbol of include/thorn_amd.h, and rejects bad input.

CPU only: nothing here launches a kernel (error paths return before any HIP call).
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from thorn_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / 'include' / 'thorn_amd.h'


def header_functions():
    text = HEADER.read_text()
    text = re.sub(r'/\*.*?\*/', '', text, flags=re.S)
    return sorted(set(re.findall(r'\b(thorn_[a-z0-9_]+)\s*\(', text)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    names = header_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f'{n} has no ctypes signature in thorn_amd/_lib.py'
    assert set(_lib.SIGNATURES) == set(names)


def test_abi_version_and_struct_sizes():
    lib = _lib.load()
    assert lib.thorn_abi_version() == _lib.ABI_VERSION
    assert lib.thorn_abi_struct_size(0) == _lib.ORTHO_MAT_DESC.itemsize
    assert lib.thorn_abi_struct_size(1) == _lib.ORTHO_MAT_STEP.itemsize
    assert lib.thorn_abi_struct_size(2) == _lib.ADAM_TENSOR_STEP.itemsize
    assert lib.thorn_abi_struct_size(3) == _lib.ADAM_SPARSE_STEP.itemsize
    assert lib.thorn_abi_struct_size(99) == 0


def test_sparse_adam_validates_without_gpu():
    """thorn_adam_sparse_step: bad records fail before any launch; nnz = 0 is a no-op."""
    rec = np.zeros(1, dtype=_lib.ADAM_SPARSE_STEP)
    with pytest.raises(_lib.ThornError, match='null argument'):
        _lib.check(_lib.load().thorn_adam_sparse_step(None, None), 'thorn_adam_sparse_step')
    rec['rows'], rec['row_len'], rec['nnz'] = 10, 4, 0
    _lib.adam_sparse_step(rec, 0)   # no rows: nothing to do
    rec['nnz'] = -1
    with pytest.raises(_lib.ThornError, match='negative size'):
        _lib.adam_sparse_step(rec, 0)
    rec['nnz'] = 3
    with pytest.raises(_lib.ThornError, match='null pointer'):
        _lib.adam_sparse_step(rec, 0)
    rec['p'], rec['m'], rec['v'], rec['g_values'], rec['g_rows'] = 4096, 8192, 12288, 16384, 20484
    with pytest.raises(_lib.ThornError, match='misaligned'):
        _lib.adam_sparse_step(rec, 0)


def test_magma_records_validate_without_gpu():
    """Magma fields (ABI 4): the scratch buffers they need are checked before any launch."""
    rec = np.zeros(1, dtype=_lib.ADAM_SPARSE_STEP)
    rec['rows'], rec['row_len'], rec['nnz'] = 10, 4, 3
    rec['p'], rec['m'], rec['v'], rec['g_values'], rec['g_rows'] = 4096, 8192, 12288, 16384, 20480
    rec['magma_s'] = 24576
    with pytest.raises(_lib.ThornError, match='needs magma_work'):
        _lib.adam_sparse_step(rec, 0)
    rec['magma_work'] = 28680
    with pytest.raises(_lib.ThornError, match='misaligned Magma'):
        _lib.adam_sparse_step(rec, 0)

    plan = _lib.AdamPlan([5000, 0, 4096])
    assert plan.workspace_bytes >= 16 * 3 and plan.workspace_bytes % 256 == 0
    steps = np.zeros(3, dtype=_lib.ADAM_TENSOR_STEP)
    for k in range(3):
        steps[k]['g'], steps[k]['m'], steps[k]['v'] = 4096, 8192, 12288
    host = np.zeros(plan.table_bytes, dtype=np.uint8)
    plan.fill_table(steps, None, 64, host.ctypes.data)   # no Magma: no workspace needed
    steps[0]['magma_s'] = 16384
    with pytest.raises(_lib.ThornError, match='needs the workspace'):
        plan.fill_table(steps, None, 64, host.ctypes.data)
    with pytest.raises(_lib.ThornError, match='256-byte aligned'):
        plan.fill_table(steps, 100, 64, host.ctypes.data)
    steps[0]['magma_s'] = 16386
    with pytest.raises(_lib.ThornError, match='magma_s must be 4-byte aligned'):
        plan.fill_table(steps, 256, 64, host.ctypes.data)

    oplan = _lib.OrthoPlan([8], [8], [0])
    osteps = np.zeros(1, dtype=_lib.ORTHO_MAT_STEP)
    osteps['p'], osteps['g'], osteps['m'], osteps['magma_s'] = 4096, 8192, 12288, 16386
    ohost = np.zeros(oplan.table_bytes, dtype=np.uint8)
    with pytest.raises(_lib.ThornError, match='magma_s must be 4-byte aligned'):
        oplan.fill_table(osteps, 256, 64, ohost.ctypes.data)


def test_w1rand_host_prng_matches_reference():
    """The product's host PRNG (Magma masks) against the reference's own sequences."""
    from thorn_amd import optim
    z = np.load(Path(__file__).resolve().parent / 'golden' / 'magma.npz')
    for seed, states, draws in zip(z['w1_seeds'], z['w1_states'], z['w1_draws']):
        st = int(seed)
        for want_s, want_d in zip(states, draws):
            st, d = optim._w1rand(st)
            assert (st, d) == (int(want_s), int(want_d))


def test_plan_rejects_bad_shapes():
    with pytest.raises(_lib.ThornError, match='unsupported shape'):
        _lib.OrthoPlan([0], [4], [0])
    with pytest.raises(_lib.ThornError, match='exclusive'):
        _lib.OrthoPlan([4], [4], [_lib.MAT_MD | _lib.MAT_MD_SCALAR])
    with pytest.raises(_lib.ThornError, match='negative'):
        _lib.AdamPlan([3, -1])
    # limits of the GEMM's and epilogues' 32-bit byte offsets
    with pytest.raises(_lib.ThornError, match=r'more than 2\^29 elements'):
        _lib.OrthoPlan([1 << 15], [1 << 14], [0])
    with pytest.raises(_lib.ThornError, match='unsupported shape'):
        _lib.OrthoPlan([2], [(1 << 20) + 1], [0])
    _lib.OrthoPlan([2], [1 << 20], [0])
    _lib.OrthoPlan([1 << 20], [2], [0])


def test_plan_sizes_and_empty_plans():
    p = _lib.OrthoPlan([1024, 3072], [1024, 1024], [0, _lib.MAT_PER_ROW_NORM])
    # two f16 iterates per matrix (the per-row-normalized u' reuses the one the last update does
    # not read); s x s f16 buffers: R and Z for the square matrix, R, Z and two Q for the tall one
    # (Gram Newton-Schulz), each its upper block triangle of 256 x 256 blocks (10 of 16 for
    # s = 1024); the per-tile partial sums add well under 1%
    want = 2 * 2 * (1024 * 1024 + 3072 * 1024) + (2 + 4) * 2 * (10 * 256 * 256)
    assert want <= p.workspace_bytes <= want * 1.01
    assert p.table_bytes > 0
    e = _lib.OrthoPlan([], [], [])
    assert e.n == 0
    a = _lib.AdamPlan([])
    assert a.table_bytes > 0


def test_fill_table_validates_pointers_without_gpu():
    plan = _lib.OrthoPlan([8], [8], [_lib.MAT_MD])
    steps = np.zeros(1, dtype=_lib.ORTHO_MAT_STEP)
    host = np.zeros(plan.table_bytes, dtype=np.uint8)
    with pytest.raises(_lib.ThornError, match='null p/g/m'):
        plan.fill_table(steps, 256, 64, host.ctypes.data)
    steps['p'] = 4096
    steps['g'] = 8192
    steps['m'] = 12288
    with pytest.raises(_lib.ThornError, match='gain state'):
        plan.fill_table(steps, 256, 64, host.ctypes.data)
    with pytest.raises(_lib.ThornError, match='256-byte aligned'):
        plan.fill_table(steps, 100, 64, host.ctypes.data)


def test_step_rejects_bad_iteration_counts():
    plan = _lib.OrthoPlan([8], [8], [0])
    with pytest.raises(_lib.ThornError, match='0 <= iters <= 32'):
        plan.step(64, np.zeros((33, 3), dtype=np.float32), 0, 0)
    # iters = 0 is a momentum-only step: refused while matrices are flagged THORN_STEP_APPLY (a
    # plan with no filled table counts as such)
    with pytest.raises(_lib.ThornError, match='momentum only'):
        plan.step(64, np.zeros((0, 3), dtype=np.float32), 0, 0)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, '_lib', None)
    monkeypatch.setattr(_lib, 'LIB_PATH', tmp_path / 'libthorn_amd.so')
    with pytest.raises(ImportError, match='no non-HIP fallback'):
        _lib.load()
