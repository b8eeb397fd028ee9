"""Where ns_phase_kernel's blocks spend one THORN step: the per-block timestamp split.

Usage (on an MI355X, after ``python -m thorn_amd.build --timestamps``)::

    python -m thorn_amd.blocksplit [--config N] [--single-chain]

It loads the measurement build (``libthorn_amd_ts.so``: the library with per-block timestamps in
``ns_phase_kernel``, see ``csrc/ns_kernels.hip``) in place of the library, runs warm-up steps of a
BASELINE workload (``bench.build_workload``), then one step whose blocks it reports:

* per kind of tile (Gram, symmetric product, update; diagonal, final): the mean prologue (block
  start to main-loop start: task lookup, operand descriptors, the first three K tiles' loads and
  the wait for tile 0), main loop (with the shader clocks per K tile), and epilogue;
* per CU: busy time out of the step's Newton-Schulz span, and the gaps between its blocks.

Timestamps are ``s_memrealtime`` (100 MHz) for times and ``s_memtime`` (shader clock) for cycles.
"""
from __future__ import annotations

import argparse
import ctypes
import sys
from collections import defaultdict
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split('\n')[0])
    ap.add_argument('--config', type=int, default=2)
    ap.add_argument('--single-chain', action='store_true', help='one plan on one stream (no chains)')
    ap.add_argument('--warmup', type=int, default=4)
    args = ap.parse_args(argv)

    sys.path.insert(0, str(ROOT))
    import torch
    from thorn_amd import _lib, build as B
    if not B.LIB_TS.exists():
        raise SystemExit(f'{B.LIB_TS} is missing: run `python -m thorn_amd.build --timestamps` first')
    _lib.LIB_PATH = B.LIB_TS
    import thorn_amd
    import bench
    if args.single_chain:
        thorn_amd.optim.CHAIN_MIN_MATRICES = 1 << 30
    lib = _lib.load()
    fetch = lib.thorn_block_timestamps
    fetch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    fetch.restype = ctypes.c_int
    slots = 262144
    buf = np.zeros(12 * slots, dtype=np.uint64)
    n = np.zeros(1, dtype=np.uint32)

    params, grads, groups, _ = bench.build_workload(args.config, 'cuda')
    opt = thorn_amd.THORN(groups)

    def step():
        for p, g in zip(params, grads):
            p.grad = g
        opt.step()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    if fetch(buf.ctypes.data, n.ctypes.data) != 0:
        raise SystemExit('thorn_block_timestamps failed')
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    step()
    e1.record()
    torch.cuda.synchronize()
    if fetch(buf.ctypes.data, n.ctypes.data) != 0:
        raise SystemExit('thorn_block_timestamps failed')
    N = int(n[0])
    if N > slots:
        raise SystemExit(f'{N} blocks: more than the {slots} slots')
    R = buf[:12 * N].reshape(N, 12).astype(np.int64)
    rs, rp, rl, re = R[:, 0], R[:, 1], R[:, 2], R[:, 3]
    cp, cl = R[:, 5], R[:, 6]
    hw, meta = R[:, 8], R[:, 9]
    xcc = (hw >> 32) & 0xF
    hwid = hw & 0xFFFFFFFF
    cuid = (((xcc * 8 + ((hwid >> 13) & 0x7)) * 2 + ((hwid >> 12) & 0x1)) * 16 + ((hwid >> 8) & 0xF))
    kind, flag, kt = meta & 0xF, (meta >> 4) & 0xF, (meta >> 8) & 0xFFFFFF
    t0 = rs.min()
    span = (re.max() - t0) / 100.0
    print(f'config {args.config}{" (one chain)" if args.single_chain else ""}: step {e0.elapsed_time(e1):.3f} ms '
          f'(measurement build); {N} ns_phase_kernel blocks over a {span:.1f} us span on {len(np.unique(cuid))} CUs')
    print('| tile | blocks | K tiles | prologue us | main loop us | cycles per K tile | epilogue us |')
    print('|---|---:|---:|---:|---:|---:|---:|')
    names = {1: 'Gram', 2: 'symmetric product', 3: 'update'}
    for k in (1, 2, 3):
        for f in (0, 1):
            m = (kind == k) & (flag == f)
            if not m.any():
                continue
            kt4 = (kt[m] + 3) // 4 * 4
            label = names[k] + ((' (diagonal)' if k != 3 else ' (final, fused apply)') if f else '')
            print(f'| {label} | {m.sum()} | {np.median(kt[m]):.0f} | {((rp[m] - rs[m]) / 100).mean():.2f} | '
                  f'{((rl[m] - rp[m]) / 100).mean():.2f} | {((cl[m] - cp[m]) / np.maximum(kt4, 1)).mean():.0f} | '
                  f'{((re[m] - rl[m]) / 100).mean():.2f} |')
    order = np.lexsort((rs, cuid))
    busy, gaps, last = defaultdict(float), defaultdict(list), {}
    for i in order:
        c = cuid[i]
        busy[c] += (re[i] - rs[i]) / 100.0
        if c in last:
            gaps[c].append((rs[i] - last[c]) / 100.0)
        last[c] = re[i]
    b = np.array(list(busy.values()))
    g = np.concatenate([np.array(v) for v in gaps.values() if v] or [np.zeros(1)])
    ncu = len(b)
    print(f'\nper CU (mean of {ncu}): busy {b.mean():.1f} of {span:.1f} us ({100 * b.mean() / span:.1f}%): '
          f'prologue {(rp - rs).sum() / 100 / ncu:.1f}, main loop {(rl - rp).sum() / 100 / ncu:.1f}, '
          f'epilogue {(re - rl).sum() / 100 / ncu:.1f} us; between blocks {g.sum() / ncu:.1f} us '
          f'(median gap {np.median(g):.2f} us)')
    clk = (R[:, 7] - R[:, 4]) / (np.maximum(re - rs, 1) * 10.0)   # cycles per ns
    print(f'mean shader clock over the blocks: {clk.mean():.2f} GHz')
    return 0


if __name__ == '__main__':
    sys.exit(main())
