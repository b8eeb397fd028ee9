"""``thorn::sym_addmm``, the reference's custom op (thorn.py:298-368), on the MI355X library.

``torch.ops.thorn.sym_addmm(A, B, C, alpha, beta)`` = beta * C + alpha * (A @ B) for products
A @ B (and C) that are symmetric: A (..., M, K), B (..., K, M), C None, (M, M) or (..., M, M);
the result is a new contiguous (..., M, M) tensor. As the reference's Triton kernel
(thorn.py:209-280), only the upper block triangle of A @ B and of C is read and computed, with
fp32 accumulation and one rounding, and the rest is its mirror. The argument checks are the
reference's (thorn.py:314-332). Float16 CUDA tensors run on the library's Newton-Schulz tiles
(thorn_sym_addmm); other dtypes and CPU tensors are refused (there is no non-HIP path).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib


def _strides(t: torch.Tensor) -> ctypes.Array:
    return (ctypes.c_int64 * 3)(*t.stride())


@torch.library.custom_op('thorn::sym_addmm', mutates_args=())
def sym_addmm(A: torch.Tensor, B: torch.Tensor, C: Optional[torch.Tensor], alpha: float,
              beta: float) -> torch.Tensor:
    assert A.device == B.device
    assert C is None or A.device == C.device
    assert A.dtype == B.dtype
    assert C is None or A.dtype == C.dtype
    assert A.ndim == B.ndim and A.ndim >= 2
    assert C is None or C.ndim >= 2
    *N, M, K = A.shape
    assert B.shape == (*N, K, M), f'B must be ({(*N, K, M)}), got {tuple(B.shape)}'
    assert C is None or C.shape[-2:] == (M, M), f'C must be (..., {M}, {M}), got {tuple(C.shape)}'
    assert C is None or C.ndim == 2 or C.shape == (*N, M, M), \
        f'C must be ({(*N, M, M)}) or ({M}, {M}), got {tuple(C.shape)}'
    NN = math.prod(N)
    assert NN <= 65535
    if not A.is_cuda or A.dtype != torch.float16:
        raise NotImplementedError(f'thorn::sym_addmm runs float16 CUDA tensors on the MI355X library; got '
                                  f'{A.dtype} on {A.device}')
    lib = _lib.load()
    A3 = A.reshape(NN, M, K)
    B3 = B.reshape(NN, K, M)
    c_mats = 0
    C3 = None
    if C is not None:
        if C.ndim == 2:
            c_mats = 1
            C3 = C.unsqueeze(0)
        else:
            c_mats = NN
            C3 = C.reshape(NN, M, M)
    out = torch.empty((NN, M, M), dtype=A.dtype, device=A.device)
    if NN == 0 or M == 0:
        return out.reshape(*N, M, M)
    with torch.cuda.device(A.device):
        nbytes = lib.thorn_sym_addmm_workspace_bytes(NN, M, K, c_mats)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=A.device)
        stream = torch.cuda.current_stream(A.device).cuda_stream
        _lib.check(lib.thorn_sym_addmm(A3.data_ptr(), _strides(A3), B3.data_ptr(), _strides(B3),
                                       C3.data_ptr() if C3 is not None else None,
                                       _strides(C3) if C3 is not None else None, c_mats, out.data_ptr(),
                                       NN, M, K, float(alpha), float(beta), ws.data_ptr(), nbytes, stream),
                   'thorn_sym_addmm')
    return out.reshape(*N, M, M)


@sym_addmm.register_fake
def _sym_addmm_fake(A, B, C, alpha, beta):
    *N, M, _ = A.shape
    return A.new_empty((*N, M, M))
