"""ctypes binding of libthorn_amd.so (the C ABI in include/thorn_amd.h).

The library is loaded after ``torch`` so that both share one HIP runtime (the library's
``libamdhip64.so.7`` dependency resolves to the copy torch already loaded). There is no fallback:
if the library is missing or fails to load, importing the optimizer's step path raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import numpy as np
import torch  # noqa: F401  (loads the HIP runtime first)

LIB_PATH = Path(__file__).resolve().parent / 'libthorn_amd.so'

THORN_OK = 0
THORN_ERR_INVALID = 1
THORN_ERR_HIP = 2
THORN_ERR_UNSUPPORTED = 3

MAT_PER_ROW_NORM = 1
MAT_MD = 2
MAT_MD_SCALAR = 4
MAT_ADAM = 8
MAT_NORM_ROWS = 16
STEP_KEEP_GRAD = 8
STEP_APPLY = 16

# numpy mirrors of the C structs (align=True reproduces the C layout on x86-64)
ORTHO_MAT_DESC = np.dtype([('rows', np.int64), ('cols', np.int64), ('flags', np.int32),
                           ('reserved', np.int32)], align=True)
ORTHO_MAT_STEP = np.dtype([
    ('p', np.uint64), ('g', np.uint64), ('m', np.uint64),
    ('row_gain', np.uint64), ('col_gain', np.uint64),
    ('row_gain_moment', np.uint64), ('row_gain_variance', np.uint64),
    ('col_gain_moment', np.uint64), ('col_gain_variance', np.uint64),
    ('target_norm', np.uint64),
    ('eta', np.float32), ('weight_decay', np.float32), ('beta1', np.float32),
    ('gain_lr', np.float32), ('gain_beta2', np.float32), ('gain_w1', np.float32),
    ('gain_w2', np.float32), ('gain_eps', np.float32),
    ('gain_bc1', np.float32), ('gain_bc2', np.float32),
    ('step_flags', np.int32), ('reserved', np.int32),
    ('magma_s', np.uint64),
    ('v', np.uint64),
    ('adam_beta2', np.float32), ('adam_w1', np.float32), ('adam_w2', np.float32),
    ('adam_bc1', np.float32), ('adam_bc2', np.float32), ('adam_eps', np.float32),
    ('adam_degenerate', np.int32), ('pnn_eps', np.float32),
], align=True)
ADAM_TENSOR_STEP = np.dtype([
    ('p', np.uint64), ('g', np.uint64), ('m', np.uint64), ('v', np.uint64),
    ('lr', np.float32), ('weight_decay', np.float32), ('beta2', np.float32),
    ('w1', np.float32), ('w2', np.float32), ('bc1', np.float32), ('bc2', np.float32),
    ('eps', np.float32), ('apply', np.int32), ('degenerate', np.int32),
    ('magma_s', np.uint64),
], align=True)

ADAM_SPARSE_STEP = np.dtype([
    ('p', np.uint64), ('m', np.uint64), ('v', np.uint64), ('g_values', np.uint64), ('g_rows', np.uint64),
    ('rows', np.int64), ('row_len', np.int64), ('nnz', np.int64),
    ('lr', np.float32), ('weight_decay', np.float32), ('beta2', np.float32),
    ('w1', np.float32), ('w2', np.float32), ('bc1', np.float32), ('bc2', np.float32),
    ('eps', np.float32), ('apply', np.int32), ('degenerate', np.int32),
    ('magma_s', np.uint64), ('magma_work', np.uint64),
], align=True)
SPARSE_MAGMA_WORK_BYTES = 16384

# every exported symbol of include/thorn_amd.h: name -> (restype, argtypes)
_vp, _sz, _i, _f, _cp = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_char_p
SIGNATURES = {
    'thorn_abi_version': (_i, []),
    'thorn_last_error': (_cp, []),
    'thorn_abi_struct_size': (_sz, [_i]),
    'thorn_ortho_plan_create': (_i, [_vp, _i, ctypes.POINTER(_vp)]),
    'thorn_ortho_plan_destroy': (None, [_vp]),
    'thorn_ortho_workspace_bytes': (_sz, [_vp]),
    'thorn_ortho_table_bytes': (_sz, [_vp]),
    'thorn_ortho_fill_table': (_i, [_vp, _vp, _vp, _vp, _vp]),
    'thorn_ortho_step': (_i, [_vp, _vp, _vp, _i, ctypes.c_uint32, _vp]),
    'thorn_ortho_step_event': (_i, [_vp, _vp, _vp, _i, ctypes.c_uint32, _vp, _vp]),
    'thorn_ortho_step_noalloc': (_i, [_vp, _vp, _vp, _i, ctypes.c_uint32, _vp]),
    'thorn_adam_plan_create': (_i, [_vp, _i, ctypes.POINTER(_vp)]),
    'thorn_adam_plan_destroy': (None, [_vp]),
    'thorn_adam_table_bytes': (_sz, [_vp]),
    'thorn_adam_workspace_bytes': (_sz, [_vp]),
    'thorn_adam_fill_table': (_i, [_vp, _vp, _vp, _vp, _vp]),
    'thorn_adam_step': (_i, [_vp, _vp, _vp]),
    'thorn_adam_sparse_step': (_i, [_vp, _vp]),
    'thorn_sym_addmm_workspace_bytes': (_sz, [ctypes.c_int64] * 4),
    'thorn_sym_addmm': (_i, [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int64,
                             ctypes.c_int64, _f, _f, _vp, _sz, _vp]),
    'thorn_ortho_timing_enable': (_i, [_vp, _i]),
    'thorn_ortho_set_spin_limit': (_i, [_vp, _i]),
    'thorn_ortho_set_small_fusion': (_i, [_vp, _i]),
    'thorn_ortho_set_small_xcd_barriers': (_i, [_vp, _i]),
    'thorn_ortho_timing_read': (_i, [_vp, _vp, _vp, _i]),
    'thorn_ortho_timing_intervals': (_i, [_vp, _vp, _vp, _vp, _vp, _i, ctypes.POINTER(_i)]),
    'thorn_adam_timing_enable': (_i, [_vp, _i]),
    'thorn_adam_timing_read': (_i, [_vp, _vp, _vp, _i]),
}
KINDS = ['pre', 'norm', 'gram', 'poly', 'update', 'rowstats', 'pnn_apply', 'md_factor', 'md_rescale', 'adam', 'cast',
         'symprod', 'magma', 'small']
WS_STATUS_OFFSET = 256
NOALLOC_SCRATCH_BYTES = 32 << 20
ABI_VERSION = 10

_lib = None


def load() -> ctypes.CDLL:
    """Loads and checks the library once; raises ImportError when it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f'{LIB_PATH} is missing: build it with `python -m thorn_amd.build` '
                          '(hipcc, gfx950). THORN has no non-HIP fallback.')
    lib = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.thorn_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f'{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it')
    for which, dt in enumerate((ORTHO_MAT_DESC, ORTHO_MAT_STEP, ADAM_TENSOR_STEP, ADAM_SPARSE_STEP)):
        size = lib.thorn_abi_struct_size(which)
        if size != dt.itemsize:
            raise ImportError(f'ABI struct {which} is {size} bytes in the library but {dt.itemsize} '
                              'in the binding; rebuild the library')
    _lib = lib
    return lib


class ThornError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != THORN_OK:
        msg = load().thorn_last_error().decode(errors='replace')
        raise ThornError(f'{what} failed (code {rc}): {msg}')


def _timing_read(fn, handle) -> dict:
    ms = np.zeros(len(KINDS), dtype=np.float64)
    cnt = np.zeros(len(KINDS), dtype=np.int32)
    check(fn(handle, ms.ctypes.data, cnt.ctypes.data, len(KINDS)), 'timing_read')
    return {k: (float(ms[i]), int(cnt[i])) for i, k in enumerate(KINDS) if cnt[i] > 0}


class OrthoPlan:
    """Host plan of one orthogonalized matrix set (shapes and per-matrix options)."""

    def __init__(self, rows, cols, flags):
        lib = load()
        self._lib = lib
        descs = np.zeros(len(rows), dtype=ORTHO_MAT_DESC)
        descs['rows'] = rows
        descs['cols'] = cols
        descs['flags'] = flags
        h = ctypes.c_void_p()
        check(lib.thorn_ortho_plan_create(descs.ctypes.data if len(rows) else None, len(rows),
                                          ctypes.byref(h)), 'thorn_ortho_plan_create')
        self.handle = h
        self.n = len(rows)
        self.workspace_bytes = lib.thorn_ortho_workspace_bytes(h)
        self.table_bytes = lib.thorn_ortho_table_bytes(h)

    def fill_table(self, steps: np.ndarray, workspace: int, table_dev: int, table_host: int) -> None:
        check(self._lib.thorn_ortho_fill_table(self.handle, steps.ctypes.data, workspace, table_dev,
                                               table_host), 'thorn_ortho_fill_table')

    def step(self, table_dev: int, coeffs: np.ndarray, restart_mask: int, stream: int,
             ns_begin_event: int = 0) -> None:
        """coeffs: (iters, 3) float32; restart_mask: bit i = restart before iteration i.
        ns_begin_event: a hipEvent_t recorded on the stream once the prologue launches are
        enqueued (thorn_ortho_step_event), or 0."""
        iters = coeffs.shape[0]
        if ns_begin_event:
            check(self._lib.thorn_ortho_step_event(self.handle, table_dev, coeffs.ctypes.data, iters, restart_mask,
                                                   stream, ns_begin_event), 'thorn_ortho_step_event')
        else:
            check(self._lib.thorn_ortho_step(self.handle, table_dev, coeffs.ctypes.data, iters, restart_mask,
                                             stream), 'thorn_ortho_step')

    def step_noalloc(self, steps: np.ndarray, coeffs: np.ndarray, restart_mask: int, stream: int) -> None:
        """fill_table + step with the library's static device workspace (no allocation)."""
        iters = coeffs.shape[0]
        check(self._lib.thorn_ortho_step_noalloc(self.handle, steps.ctypes.data, coeffs.ctypes.data, iters,
                                                 restart_mask, stream), 'thorn_ortho_step_noalloc')

    def timing_enable(self, max_launches: int) -> None:
        check(self._lib.thorn_ortho_timing_enable(self.handle, max_launches), 'thorn_ortho_timing_enable')

    def set_spin_limit(self, polls: int) -> None:
        check(self._lib.thorn_ortho_set_spin_limit(self.handle, polls), 'thorn_ortho_set_spin_limit')

    def set_small_fusion(self, enable: bool) -> None:
        check(self._lib.thorn_ortho_set_small_fusion(self.handle, int(bool(enable))), 'thorn_ortho_set_small_fusion')

    def set_small_xcd_barriers(self, enable: bool) -> None:
        check(self._lib.thorn_ortho_set_small_xcd_barriers(self.handle, int(bool(enable))),
              'thorn_ortho_set_small_xcd_barriers')

    def timing_read(self) -> dict:
        return _timing_read(self._lib.thorn_ortho_timing_read, self.handle)

    def timing_intervals(self, ref_event: int, max_launches: int) -> list:
        """[(kind name, start ms, end ms)] of the recorded launches, relative to ref_event (a
        timing-enabled hipEvent recorded before them); starts a new window."""
        s = np.zeros(max(1, max_launches), dtype=np.float64)
        e = np.zeros_like(s)
        k = np.zeros(max(1, max_launches), dtype=np.int32)
        n = ctypes.c_int(0)
        check(self._lib.thorn_ortho_timing_intervals(self.handle, ref_event, s.ctypes.data, e.ctypes.data,
                                                     k.ctypes.data, max_launches, ctypes.byref(n)),
              'thorn_ortho_timing_intervals')
        return [(KINDS[k[i]] if 0 <= k[i] < len(KINDS) else str(k[i]), float(s[i]), float(e[i]))
                for i in range(n.value)]

    def __del__(self):
        h = getattr(self, 'handle', None)
        if h is not None and h.value:
            self._lib.thorn_ortho_plan_destroy(h)
            self.handle = None


class AdamPlan:
    """Host plan of one multi-tensor Adam launch (element counts of every tensor)."""

    def __init__(self, numels):
        lib = load()
        self._lib = lib
        arr = np.asarray(numels, dtype=np.int64)
        h = ctypes.c_void_p()
        check(lib.thorn_adam_plan_create(arr.ctypes.data if len(arr) else None, len(arr), ctypes.byref(h)),
              'thorn_adam_plan_create')
        self.handle = h
        self.n = len(arr)
        self.table_bytes = lib.thorn_adam_table_bytes(h)
        self.workspace_bytes = lib.thorn_adam_workspace_bytes(h)

    def fill_table(self, steps: np.ndarray, workspace: Optional[int], table_dev: int, table_host: int) -> None:
        check(self._lib.thorn_adam_fill_table(self.handle, steps.ctypes.data, workspace, table_dev, table_host),
              'thorn_adam_fill_table')

    def step(self, table_dev: int, stream: int) -> None:
        check(self._lib.thorn_adam_step(self.handle, table_dev, stream), 'thorn_adam_step')

    def timing_enable(self, max_launches: int) -> None:
        check(self._lib.thorn_adam_timing_enable(self.handle, max_launches), 'thorn_adam_timing_enable')

    def timing_read(self) -> dict:
        return _timing_read(self._lib.thorn_adam_timing_read, self.handle)

    def __del__(self):
        h = getattr(self, 'handle', None)
        if h is not None and h.value:
            self._lib.thorn_adam_plan_destroy(h)
            self.handle = None


def adam_sparse_step(step: np.ndarray, stream: int) -> None:
    """step: one ADAM_SPARSE_STEP record (see include/thorn_amd.h)."""
    assert step.dtype == ADAM_SPARSE_STEP and step.size == 1
    check(load().thorn_adam_sparse_step(step.ctypes.data, stream), 'thorn_adam_sparse_step')
