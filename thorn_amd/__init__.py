"""THORN optimizer step on AMD Instinct MI355X (gfx950).

``from thorn_amd import THORN`` is a drop-in for ``from thorn import THORN`` (pykeio/THORN): same
constructor, parameter groups, state layout and ``step``. The step runs as hand-written HIP
kernels in ``libthorn_amd.so`` (C ABI: include/thorn_amd.h); there is no CPU or PyTorch-op
fallback.
"""
from . import ops  # registers the thorn::sym_addmm custom op (thorn.py:298)
from .optim import THORN, THORNGroup, THORNNonOrthoGroup, THORNOrthoGroup

__version__ = '3.1.1'
__all__ = ['THORN', 'THORNOrthoGroup', 'THORNNonOrthoGroup', 'THORNGroup']
