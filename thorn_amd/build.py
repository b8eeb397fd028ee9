"""Builds the gfx950 THORN library (thorn_amd/libthorn_amd.so) with hipcc.

Usage: ``python -m thorn_amd.build`` (also called by ``__graft_entry__.build()``).
The library is a single translation unit, ``csrc/thorn_abi.hip``, exporting the C ABI declared in
``include/thorn_amd.h``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / 'csrc' / 'thorn_abi.hip'
LIB = PKG / 'libthorn_amd.so'
ARCH = 'gfx950'

HIPCC_FLAGS = [
    f'--offload-arch={ARCH}',
    '-O3',
    '-std=c++17',
    '-fPIC',
    '-shared',
    # every multiply and add rounds on its own, like PyTorch's eager ops; fmaf is explicit
    '-ffp-contract=off',
    # no packed fp32 instructions (v_pk_*_f32) in any kernel
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wno-unused-result',
]


def hipcc() -> str:
    exe = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(exe):
        raise RuntimeError('hipcc not found; the THORN library needs ROCm to build')
    return exe


# The measurement build: the same library with per-block timestamps in ns_phase_kernel
# (`python -m thorn_amd.blocksplit`); never loaded by THORN itself.
LIB_TS = PKG / 'libthorn_amd_ts.so'


def build(verbose: bool = False, timestamps: bool = False) -> Path:
    """Compiles the library (timestamps: the measurement build) in place and returns its path
    (always rebuilds)."""
    out = LIB_TS if timestamps else LIB
    tmp = out.with_suffix('.so.tmp')
    cmd = [hipcc(), *HIPCC_FLAGS, *(['-DTHORN_BLOCK_TIMESTAMPS'] if timestamps else []), f'-I{ROOT / "include"}',
           str(SRC), '-o', str(tmp)]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}')
    os.replace(tmp, out)
    return out


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv, timestamps='--timestamps' in sys.argv))
