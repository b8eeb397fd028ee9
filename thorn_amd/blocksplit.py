"""Where ns_phase_kernel's blocks spend one THORN step: the per-block timestamp split.

Usage (on an MI355X, after ``python -m thorn_amd.build --timestamps``)::

    python -m thorn_amd.blocksplit [--config N] [--single-chain] [--separate]

It loads the measurement build (``libthorn_amd_ts.so``: the library with per-block timestamps in
``ns_phase_kernel``, see ``csrc/ns_kernels.hip``) in place of the library, runs warm-up steps of a
BASELINE workload (``bench.build_workload``), then one step whose blocks it reports:

* per kind of tile (Gram, symmetric product, update; diagonal, final): the mean prologue (block
  start to main-loop start: task lookup, operand descriptors, the first three K tiles' loads and
  the wait for tile 0), main loop (with the shader clocks per K tile), and epilogue;
* per CU: busy time out of the step's Newton-Schulz span, and the gaps between its blocks;
* for ``ns_small_kernel`` (matrices with a short side of at most 256), per matrix: its cluster of
  workgroups and their prologue (the fused step's momentum, norm and first iterate), schedule and
  epilogue (the fused step's update of p), from the launch's first workgroup start.

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
    ap.add_argument('--separate', action='store_true',
                    help='small-matrix plans without the fused step (thorn_ortho_set_small_fusion(plan, 0))')
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
    lib.thorn_small_op_timestamps.argtypes = [ctypes.c_void_p]
    lib.thorn_small_op_timestamps.restype = ctypes.c_int
    slots = 262144
    buf = np.zeros(12 * slots, dtype=np.uint64)
    n = np.zeros(1, dtype=np.uint32)

    params, grads, groups, _ = bench.build_workload(args.config, 'cuda')
    opt = thorn_amd.THORN(groups)

    def step():
        for p, g in zip(params, grads):
            p.grad = g
        opt.step()
    for w in range(max(1, args.warmup)):
        step()
        if w == 0 and args.separate:   # the plans exist after the first step
            for r in opt._runners.values():
                for pl in r.plans:
                    if isinstance(pl, _lib.OrthoPlan):
                        pl.set_small_fusion(False)
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
    small = kind == 4
    if small.any():
        shapes = [(r, c) for grp in opt.param_groups if grp['orthogonalize']
                  for r, c in zip(*thorn_amd.optim._plan_shapes(grp['params'],
                                                                thorn_amd.optim._Group.from_kwargs(**grp), False)[:2])]
        s0 = rs[small].min()
        print(f'ns_small_kernel ({"fused step" if flag[small].max() else "schedule only"}): '
              f'{small.sum()} workgroups, {(re[small].max() - s0) / 100:.1f} us from the first start to the last end')
        print('| matrix | workgroups | start us | prologue us | schedule us | epilogue us | end us |')
        print('|---|---:|---:|---:|---:|---:|---:|')
        mat = (meta >> 20) & 0xFFF
        for i in sorted(set(mat[small].tolist())):
            m = small & (mat == i)
            shape = shapes[i] if i < len(shapes) else '?'
            print(f'| {shape} | {m.sum()} | {(rs[m].min() - s0) / 100:.1f} | {((rp[m] - rs[m]) / 100).max():.1f} | '
                  f'{((rl[m] - rp[m]) / 100).max():.1f} | {((re[m] - rl[m]) / 100).max():.1f} | '
                  f'{(re[m].max() - s0) / 100:.1f} |')
        # the last cluster to finish: per operation, from the first member's start to the last
        # member's products, its stores, and the barrier until the last member starts the next one
        sop = np.zeros(4096 * 64 * 5, dtype=np.uint64)
        if lib.thorn_small_op_timestamps(sop.ctypes.data) == 0:
            sop = sop.reshape(4096, 64, 5).astype(np.int64)
            crit = int(mat[small][np.argmax(re[small])])
            rows_ = [i for i in np.nonzero(small & (mat == crit))[0] if i < 4096]
            ops = sop[rows_]                      # members x 64 x 3
            nops = int(((ops[:, :, 0] >= rs[rows_, None]) & (ops[:, :, 0] <= re[rows_, None])).all(axis=0).sum())
            print(f'\n{shapes[crit] if crit < len(shapes) else crit}, per operation (us): products (first K chunk '
                  'landed + K loop + end) | stores | barrier to the next operation')
            line = []
            for q in range(nops):
                st, pr, sd = ops[:, q, 0].min(), ops[:, q, 1].max(), ops[:, q, 2].max()
                # members with a super-tile in this operation (the others keep older stamps)
                w = (ops[:, q, 3] >= ops[:, q, 0]) & (ops[:, q, 3] <= ops[:, q, 2])
                f0 = (ops[w, q, 3] - ops[w, q, 0]).mean() / 100 if w.any() else 0.0
                lp = (ops[w, q, 4] - ops[w, q, 3]).mean() / 100 if w.any() else 0.0
                nxt = ops[:, q + 1, 0].max() if q + 1 < nops else rl[rows_].max()
                line.append(f'{q}: {(pr - st) / 100:.1f} ({f0:.1f} + {lp:.1f} + {(pr - st) / 100 - f0 - lp:.1f}) | '
                            f'{(sd - pr) / 100:.1f} | {(nxt - sd) / 100:.1f}')
            print('; '.join(line))
        keep = ~small
        if not keep.any():
            return 0
        R, rs, rp, rl, re, cp, cl, hw, meta = (R[keep], rs[keep], rp[keep], rl[keep], re[keep], cp[keep], cl[keep],
                                               hw[keep], meta[keep])
        kind, flag, kt, N = kind[keep], flag[keep], kt[keep], int(keep.sum())
        xcc = (hw >> 32) & 0xF
        hwid = hw & 0xFFFFFFFF
        cuid = (((xcc * 8 + ((hwid >> 13) & 0x7)) * 2 + ((hwid >> 12) & 0x1)) * 16 + ((hwid >> 8) & 0xF))
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
