#!/usr/bin/env python
"""THORN step benchmark on one MI355X (BASELINE.json metric: step ms on the Qwen3 ~300M set).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu-baseline]

Workload (synthetic, seed 3407, generated on the CPU and copied to HBM):
20 layers x {q 2048x1024, k 1024x1024, v 1024x1024, o 1024x2048, gate 3072x1024, up 3072x1024,
down 1024x3072} (orthogonalized, wd 0.1, moonlight), 41 RMSNorm vectors of 1024 (wd 0) and a
151936x1024 embedding (wd 0.1); params N(0, 0.02), grads N(0, 1e-3^2) with 1% of rows x10. A
"step" is one full ``optimizer.step()`` over all of it (momentum, 5 Newton-Schulz iterations,
per-row normalization, cautious weight decay, Adam); inputs are resident in HBM, and each step
re-attaches the pre-drawn gradients (``none_grad=True`` frees them).

Prints one JSON line: step ms (value, lower is better), the Newton-Schulz TFLOP/s against the
f16/bf16 dense MFMA peak, the update kernels' GB/s against HBM, a per-kernel breakdown measured
with HIP events on the launch stream, and the CPU baseline (the oracle, a restatement of the
reference's eager CPU path, timed on this host on a bounded sample and scaled to a full step).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_PEAK_TFLOPS = 2500.0   # MI355X dense f16/bf16 MFMA
HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E
# Plan kinds of the Newton-Schulz launches, and the small-matrix path's limits (thorn_abi.hip)
NS_KINDS = ('gram', 'poly', 'symprod', 'update', 'small')
SMALL_MAX_S, SMALL_MAX_ELEMS = 256, 1 << 20


# ---------------------------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------------------------

def config_shapes(config: int):
    """(ortho matrix shapes, non-ortho groups [(shape list, wd)], group overrides)."""
    if config == 1:
        return [(512, 256)], []
    if config in (2, 3):
        layer = [(2048, 1024), (1024, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (3072, 1024), (1024, 3072)]
        return layer * 20, [([(151936, 1024)], 0.1), ([(1024,)] * 41, 0.0)]
    if config == 4:
        mats = [(32, 5), (64, 96), (64, 192), (128, 192), (128, 384), (256, 640), (256, 128)]
        vecs = [(n,) for n in [32, 64, 64, 128, 128, 256] * 2]
        return mats, [(vecs, 0.0)]
    if config == 5:
        layer = [(2048, 2048), (1024, 2048), (1024, 2048), (2048, 2048), (6144, 2048), (6144, 2048), (2048, 6144)]
        return layer * 28 + [(8192, 8192), (16384, 1024)], []
    raise SystemExit(f'unknown config {config}')


def ns_flops(shapes, iters=5) -> float:
    """Plain-quintic algorithmic flops: iters * (3 s^2 l + s^3), symmetric products counted once."""
    total = 0.0
    for r, c in shapes:
        s, l = min(r, c), max(r, c)
        total += iters * (3.0 * s * s * l + s ** 3)
    return total


def gram_ops(iters: int, restart_mask: int) -> list:
    """The Gram Newton-Schulz operations the library launches for one non-square matrix
    (thorn_abi.hip, gram_schedule; the reference's recurrences, thorn.py:637-653): 'gram'
    (R = X X^T), 'poly' (Z = b R + c R^2), 'sym' (a Q + Q Z, a R + R Z, a RZ + Z RZ) and 'update'
    (Q X)."""
    def restart(i):
        return 0 < i < 32 and (restart_mask >> i) & 1
    ops = ['gram']
    for i in range(iters):
        if restart(i):
            ops += ['update', 'gram']
        ops.append('poly')
        if i != 0 and not restart(i):
            ops.append('sym')
        if i < iters - 1 and not restart(i + 1):
            ops += ['sym', 'sym']
    ops.append('update')
    return ops


def plain_ops(iters: int) -> list:
    """The plain quintic for one square matrix (thorn.py:654-658): A = X X^T, B = b A + c A^2,
    X <- a X + B X per iteration (thorn_abi.hip, plain_schedule)."""
    return ['gram', 'poly', 'update'] * iters


def op_counts(ops: list) -> dict:
    return {k: ops.count(k) for k in ('gram', 'poly', 'sym', 'update')}


def schedule_flops(shapes, iters: int, restart_mask: int) -> float:
    """Algorithmic flops of the schedules the library runs: Gram Newton-Schulz with `restart_mask`
    on every non-square matrix, the plain quintic on square ones (thorn.py:628); s^2 l per Gram
    matrix, s^3 per polynomial or symmetric product (symmetric results counted once), 2 s^2 l per
    update. For square matrices this is ns_flops."""
    plain = op_counts(plain_ops(iters))
    gram = op_counts(gram_ops(iters, restart_mask))
    total = 0.0
    for r, c in shapes:
        s, l = min(r, c), max(r, c)
        sched = gram if r != c else plain
        total += (sched['gram'] * s * s * l + (sched['poly'] + sched['sym']) * s ** 3
                  + sched['update'] * 2.0 * s * s * l)
    return total


def build_workload(config: int, device):
    """Parameters and gradients drawn on the CPU from seed 3407 (params first, then grads), moved
    to `device` bit for bit."""
    import torch
    gen = torch.Generator().manual_seed(3407)
    mats, others = config_shapes(config)
    scale_p = 0.05 if config == 4 else 0.02
    scale_g = 1e-2 if config == 4 else 1e-3
    p_cpu = []
    for sh in mats:
        p_cpu.append(torch.randn(sh, generator=gen) * scale_p)
    for shapes, _ in others:
        for sh in shapes:
            p_cpu.append(torch.ones(sh) if len(sh) == 1 else torch.randn(sh, generator=gen) * scale_p)
    g_cpu = []
    for t in p_cpu:
        if config == 5:
            # Student-t(3) noise at the same scale
            z = torch.randn(t.shape, generator=gen)
            chi = sum(torch.randn(t.shape, generator=gen) ** 2 for _ in range(3))
            g = z / torch.sqrt(chi / 3) * scale_g
        else:
            g = torch.randn(t.shape, generator=gen) * scale_g
        if t.ndim == 2 and config in (2, 3):
            k = max(1, round(0.01 * t.shape[0]))
            rows = torch.randperm(t.shape[0], generator=gen)[:k]
            g[rows] *= 10.0
        g_cpu.append(g)
    params = [torch.nn.Parameter(t.to(device)) for t in p_cpu]
    grads = [g.to(device) for g in g_cpu]
    n_m = len(mats)
    groups = [{'orthogonalize': True, 'params': params[:n_m], 'lr': 1e-3, 'betas': (0.9, 0.95),
               'weight_decay': 0.1, 'scaling_mode': 'moonlight'}]
    if config == 3:
        groups[0].update(lr=8e-3, weight_decay=0.0, decouple_md=True)
        del groups[0]['scaling_mode']
    off = n_m
    for shapes, wd in others:
        groups.append({'orthogonalize': False, 'params': params[off:off + len(shapes)], 'lr': 1e-3,
                       'betas': (0.9, 0.95), 'weight_decay': wd})
        off += len(shapes)
    return params, grads, groups, mats


def compulsory_bytes(mats, params, n_m) -> float:
    """20 B per orthogonalized element (g, m read; m write; p read, write); 28 B per Adam element."""
    ortho = sum(r * c for r, c in mats)
    adam = sum(p.numel() for p in params[n_m:])
    return 20.0 * ortho + 28.0 * adam


# ---------------------------------------------------------------------------------------------
# CPU baseline: the oracle (restated reference eager path) on a bounded sample
# ---------------------------------------------------------------------------------------------

def host_cpu() -> dict:
    """The host's CPU model, the ISA flags that decide CPU f16 GEMM speed, and the threads used."""
    info = {'model': 'unknown', 'flags': [], 'threads': len(os.sched_getaffinity(0))}
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name') and info['model'] == 'unknown':
                info['model'] = line.split(':', 1)[1].strip()
            elif line.startswith('flags'):
                have = set(line.split(':', 1)[1].split())
                info['flags'] = sorted(f for f in ('avx2', 'avx512f', 'avx512_bf16', 'avx512_fp16', 'amx_bf16',
                                                   'amx_fp16', 'amx_tile') if f in have)
                break
    except OSError:
        pass
    return info


def gemm_probe(m: int = 256, k: int = 768, n: int = 256) -> dict:
    """torch.baddbmm GFLOP/s on the CPU in f16, bf16 and f32 at one (m x k) (k x n) product: the
    rate of the GEMMs the oracle (the reference's eager path) runs, which the host ISA decides."""
    import torch
    out = {'shape': f'{m}x{k}x{n}'}
    gen = torch.Generator().manual_seed(0)
    for name, dt in (('f16', torch.float16), ('bf16', torch.bfloat16), ('f32', torch.float32)):
        a = torch.randn(1, m, k, generator=gen).to(dt)
        b = torch.randn(1, k, n, generator=gen).to(dt)
        c = torch.zeros(1, m, n, dtype=dt)
        torch.baddbmm(c, a, b)   # warm-up
        reps, t0 = 0, time.perf_counter()
        while reps < 3 or time.perf_counter() - t0 < 0.2:
            torch.baddbmm(c, a, b)
            reps += 1
            if time.perf_counter() - t0 > 2.0:
                break
        out[name + '_gflops'] = round(2.0 * m * k * n * reps / (time.perf_counter() - t0) / 1e9, 2)
    return out


def cpu_baseline(config: int, budget_s: float = 300.0) -> dict:
    """The oracle (the reference's eager algorithm, oracle/thorn_oracle.py) timed on this host.

    Per distinct matrix shape of the workload, cheapest first: one oracle step on one matrix of
    that shape, timed when the f16 GEMM probe (scaled by the measured-to-predicted ratio of the
    shapes already timed) predicts it fits the remaining budget ('measured'; config 2's five shapes
    take about 4 minutes on a 16-thread EPYC share, each reported on stderr as it ends);
    otherwise its time is the shape's schedule flops at the probe's f16 rate, times the ratio of
    measured to probe-predicted time of the measured shapes, or of a 256 x 768 proxy matrix when
    none was measured ('probe-scaled'). Each shape's time is multiplied by its count. The Adam
    tensors are timed on a slice (at least 1 Mi elements) and scaled by element count."""
    import torch
    from oracle import thorn_oracle as O

    host = host_cpu()
    threads = host['threads']
    torch.set_num_threads(threads)
    probe = gemm_probe()
    rate = probe['f16_gflops'] * 1e9   # flop/s of the oracle's f16 products
    gen = torch.Generator().manual_seed(3407)
    mats, others = config_shapes(config)
    counts = {}
    for sh in mats:
        counts[sh] = counts.get(sh, 0) + 1
    t_start = time.perf_counter()

    def ref_flops(sh):   # Gram NS (restart before iteration 2) if non-square, else the plain quintic
        return schedule_flops([sh], 5, 0b100)

    def one_step(sh):
        p = torch.nn.Parameter(torch.randn(sh, generator=gen) * 0.02)
        opt = O.OracleTHORN([{'orthogonalize': True, 'params': [p], 'lr': 1e-3, 'weight_decay': 0.1,
                              'scaling_mode': 'moonlight'}])
        p.grad = torch.randn(sh, generator=gen) * 1e-3
        t0 = time.perf_counter()
        opt.step()
        return time.perf_counter() - t0

    per_shape, ratios = {}, []
    for sh in sorted(counts, key=ref_flops):
        predicted = ref_flops(sh) / rate
        scale = sorted(ratios)[len(ratios) // 2] if ratios else 1.0
        left = budget_s - (time.perf_counter() - t_start)
        if predicted * scale < left:
            t = one_step(sh)
            ratios.append(t / predicted)
            print(f'cpu_baseline: {sh[0]}x{sh[1]} one oracle step {t:.1f} s', file=sys.stderr, flush=True)
            per_shape[sh] = {'count': counts[sh], 'gflop': round(ref_flops(sh) / 1e9, 2), 's': round(t, 3),
                             'how': 'measured'}
    if not ratios:   # calibrate on a proxy with the workload's most common aspect ratio
        proxy = (256, 768)
        ratios.append(one_step(proxy) / (ref_flops(proxy) / rate))
    ratio = sorted(ratios)[len(ratios) // 2]
    for sh in counts:
        if sh not in per_shape:
            per_shape[sh] = {'count': counts[sh], 'gflop': round(ref_flops(sh) / 1e9, 2),
                             's': round(ref_flops(sh) / rate * ratio, 3), 'how': 'probe-scaled'}
    est = sum(v['count'] * v['s'] for v in per_shape.values())
    adam_total = sum(math.prod(sh) for shapes, _ in others for sh in shapes)
    adam = None
    if adam_total:
        n_slice = min(max(1 << 20, adam_total // 10), adam_total)
        p = torch.nn.Parameter(torch.randn(n_slice, generator=gen) * 0.02)
        opt = O.OracleTHORN([{'orthogonalize': False, 'params': [p], 'lr': 1e-3, 'weight_decay': 0.1}])
        ts = []
        for _ in range(3):
            p.grad = torch.randn(n_slice, generator=gen) * 1e-3
            t0 = time.perf_counter()
            opt.step()
            ts.append(time.perf_counter() - t0)
        adam_s = sorted(ts)[1] * adam_total / n_slice
        adam = {'elements': adam_total, 'sampled': n_slice, 's': round(adam_s, 3)}
        est += adam_s
    n_meas = sum(v['how'] == 'measured' for v in per_shape.values())
    return {
        'value': round(est * 1000.0, 1), 'unit': 'ms per full step', 'cores': threads, 'kind': 'port',
        'sample': (f'{n_meas}/{len(per_shape)} shapes measured'
                   + ('' if n_meas == len(per_shape) else ', rest probe-scaled')
                   + f' (one oracle step on one matrix of each, times its count); Adam sliced; '
                   f'{time.perf_counter() - t_start:.0f} s'),
        'host': host, 'gemm_probe': probe, 'probe_to_oracle_ratio': round(ratio, 3),
        'per_shape': {f'{r}x{c}': v for (r, c), v in per_shape.items()}, 'adam': adam,
    }


# ---------------------------------------------------------------------------------------------
# rocprofv3 summaries and the HBM-traffic calibration
# ---------------------------------------------------------------------------------------------

TRAFFIC_PROFILES = {'ns_phase_kernel': 'ns_phase_traffic_qwen3_300m.md'}


def copy_calibration(mib: int, device) -> None:
    """One plain fp32 elementwise kernel (torch.neg) over `mib` MiB: it reads and writes exactly
    `mib` MiB, so what FETCH_SIZE / WRITE_SIZE report for it gives the counters' scale."""
    import torch
    src = torch.ones(mib << 18, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def _short_kernel_name(name: str) -> str:
    import re
    name = re.sub(r'^void ', '', name)
    depth, out = 0, []
    for ch in name:          # drop argument lists, keep template arguments
        if ch == '(':
            depth += 1
        elif ch == ')':
            depth -= 1
        elif depth == 0:
            out.append(ch)
    return ''.join(out).strip()


def rocprof_summary(paths: list, cal_mib: int = 0, steps: int = 5, config: int = 2) -> str:
    """Markdown summary of rocprofv3 CSV output directories: the kernel statistics table
    (`*kernel_stats.csv`) and, when present, per-kernel counter averages per dispatch
    (`*counter_collection.csv`, one directory per counter pass). With `cal_mib`, FETCH_SIZE /
    WRITE_SIZE are scaled by what they read for the `torch.neg` calibration kernel of that many
    MiB, and the HBM bytes per ns_phase_kernel launch are printed."""
    import csv
    import glob

    def found(pattern):
        return sorted(f for p in paths for f in glob.glob(os.path.join(p, '**', pattern), recursive=True))

    lines = []
    traces = found('*kernel_trace.csv')
    if traces:
        lines += ns_trace_lines(traces[0], steps, config)
    for f in found('*kernel_stats.csv'):
        rows = list(csv.DictReader(open(f)))
        lines += ['| kernel | calls | total ms | avg us | min us | max us | % |',
                  '|---|---:|---:|---:|---:|---:|---:|']
        for r in rows:
            n = _short_kernel_name(r['Name'])
            n = n if len(n) <= 70 else n[:67] + '...'
            lines.append(f"| `{n}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
                         f"{float(r['AverageNs']) / 1e3:.1f} | {float(r['MinNs']) / 1e3:.1f} | "
                         f"{float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f} |")
    per: dict = {}
    for f in found('*counter_collection.csv'):
        for r in csv.DictReader(open(f)):
            key = (_short_kernel_name(r['Kernel_Name']), r['Counter_Name'])
            per.setdefault(key, {})[(f, r['Dispatch_Id'])] = float(r['Counter_Value'])
    if per:
        counters = sorted({c for _, c in per})
        kernels = sorted({k for k, _ in per})
        scale = {}
        for c in ('FETCH_SIZE', 'WRITE_SIZE'):
            cal = [v for (k, cc), d in per.items() if cc == c and 'neg_kernel' in k for v in d.values()]
            if cal_mib and cal:
                scale[c] = cal_mib * 1024.0 / max(cal)      # KiB expected / KiB read
        lines += ['', '| kernel | dispatches | ' + ' | '.join(f'{c} / dispatch' for c in counters) + ' |',
                  '|---|---:|' + '---:|' * len(counters)]
        for k in kernels:
            vals = [per.get((k, c), {}) for c in counters]
            nd = max(len(v) for v in vals)
            cells = [f'{sum(v.values()) / len(v):.4g}' if v else '' for v in vals]
            kk = k if len(k) <= 70 else k[:67] + '...'
            lines.append(f'| `{kk}` | {nd} | ' + ' | '.join(cells) + ' |')
        if scale:
            lines += ['', 'Counter scale from the calibration kernel (expected KiB / counted KiB): ' +
                      ', '.join(f'{c} x{s:.4f}' for c, s in scale.items())]
            upd = [k for k in kernels if k.startswith('thorn::ns_phase_kernel')]
            tot = 0.0
            for c, s in scale.items():
                v = [x for k in upd for x in per.get((k, c), {}).values()]
                if v:
                    tot += sum(v) / len(v) * 1024.0 * s
            if upd and len(scale) == 2:
                lines.append(f'\nns_phase_kernel HBM bytes per launch: {tot:.6g}')
        lines += mfma_lines(found)
    return '\n'.join(lines)


def _union_us(iv: list) -> float:
    """Length of the union of (start, end) intervals."""
    total, end = 0.0, None
    for a, b in sorted(iv):
        if end is None or a > end:
            total += b - a
            end = b
        elif b > end:
            total += b - end
            end = b
    return total


def ns_trace_lines(path: str, steps: int = 5, config: int = 2) -> list:
    """From a rocprofv3 kernel trace of a config-2 bench.py run: ns_phase_kernel's launches in the
    last `steps` steps (the event-timed pass of `bench.py --steps <steps>`), as summed durations
    and as the union of their intervals, which is what bench.py reports (a group stepping as two
    chains on two streams overlaps them); with one stream, also the Newton-Schulz launches of the
    last complete step, op by op. A stream's steps begin at its ortho_pre_kernel launches."""
    import csv
    rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r['Start_Timestamp']))
    iv = lambda r: (int(r['Start_Timestamp']) / 1e3, int(r['End_Timestamp']) / 1e3)
    per_stream: dict = {}
    for r in rows:
        per_stream.setdefault(r['Stream_Id'], []).append(r)
    pre = {k: [i for i, r in enumerate(v) if 'ortho_pre_kernel' in r['Kernel_Name']] for k, v in per_stream.items()}
    chains = {k: v for k, v in pre.items()
              if any('ns_phase_kernel' in r['Kernel_Name'] for r in per_stream[k])}
    if not chains or min(len(v) for v in chains.values()) < steps:
        return []
    t0 = min(iv(per_stream[k][v[-steps]])[0] for k, v in chains.items())
    ns = [iv(r) for r in rows if 'ns_phase_kernel' in r['Kernel_Name'] and iv(r)[0] >= t0]
    out = [f'ns_phase_kernel in the last {steps} steps ({len(chains)} stream(s)): {len(ns) // steps} launches '
           f'per step; summed durations {sum(b - a for a, b in ns) / len(ns):.1f} us per launch; union of '
           f'their intervals {_union_us(ns) / steps / 1e3:.3f} ms per step, {_union_us(ns) / len(ns):.1f} us '
           'per launch', '']
    if len(chains) != 1:
        return out
    (k, starts), = chains.items()
    seg = [iv(r) for r in per_stream[k][starts[-2]:starts[-1]] if 'ns_phase_kernel' in r['Kernel_Name']]
    mats, _ = config_shapes(config)
    mats = [sh for sh in mats if not (min(sh) <= SMALL_MAX_S and sh[0] * sh[1] < SMALL_MAX_ELEMS)]
    gram = gram_ops(5, 4)
    plain = plain_ops(5)
    n_sq = sum(1 for sh in mats if sh[0] == sh[1])
    fl = {'gram': lambda s_, l_: s_ * s_ * l_, 'poly': lambda s_, l_: s_ ** 3,
          'sym': lambda s_, l_: s_ ** 3, 'update': lambda s_, l_: 2.0 * s_ * s_ * l_}
    out += [f'Newton-Schulz launches of the last complete step (config {config}; Gram-schedule op on the '
            f'{len(mats) - n_sq} non-square matrices / plain-schedule op on the {n_sq} square ones):', '',
            '| launch | ops | TFLOP (algorithmic) | us | TFLOP/s |', '|---:|---|---:|---:|---:|']
    for j, (a, b) in enumerate(seg):
        f = 0.0
        names = []
        for sched, pick in ((gram, lambda s_, l_: l_ != s_), (plain, lambda s_, l_: l_ == s_)):
            op = sched[j] if j < len(sched) else None
            names.append(op or '-')
            if op:
                f += sum(fl[op](min(sh), max(sh)) for sh in mats if pick(min(sh), max(sh)))
        out.append(f'| {j + 1} | {names[0]} / {names[1]} | {f / 1e12:.3f} | {b - a:.1f} | '
                   f'{f / ((b - a) * 1e-6) / 1e12:.1f} |')
    return out + ['']


def mfma_lines(found) -> list:
    """ns_phase_kernel's MFMA utilisation, clock and executed MFMA flops from the counter passes
    SQ_VALU_MFMA_BUSY_CYCLES + GRBM_GUI_ACTIVE and SQ_INSTS_VALU_MFMA_MOPS_F16 (one 512-flop op
    each), per dispatch, with the dispatch's own start/end timestamps. GRBM_GUI_ACTIVE comes summed
    over the XCDs, so a dispatch's cycles are it / Num_Xcc; MfmaUtil = busy / (cycles * Simd_Count),
    as rocprofv3's derived metric defines it."""
    import csv
    agent = [r for f in found('*agent_info.csv') for r in csv.DictReader(open(f)) if r['Agent_Type'] == 'GPU']
    if not agent:
        return []
    xcc, simds = int(agent[0]['Num_Xcc']), int(agent[0]['Simd_Count'])
    fmax = float(agent[0]['Max_Engine_Clk_Fcompute'])
    per: dict = {}
    for f in found('*counter_collection.csv'):
        for r in csv.DictReader(open(f)):
            if 'ns_phase_kernel' not in r['Kernel_Name']:
                continue
            d = per.setdefault((f, r['Dispatch_Id']), {})
            d[r['Counter_Name']] = float(r['Counter_Value'])
            d['ns'] = int(r['End_Timestamp']) - int(r['Start_Timestamp'])
    util, clk, rate = [], [], []
    for d in per.values():
        if 'SQ_VALU_MFMA_BUSY_CYCLES' in d and 'GRBM_GUI_ACTIVE' in d:
            cyc = d['GRBM_GUI_ACTIVE'] / xcc
            util.append(d['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * simds))
            clk.append(cyc / d['ns'])
        if 'SQ_INSTS_VALU_MFMA_MOPS_F16' in d:
            rate.append(d['SQ_INSTS_VALU_MFMA_MOPS_F16'] * 512 / d['ns'] / 1e3)   # TFLOP/s
    if not (util or rate):
        return []
    avg = lambda v: sum(v) / len(v)
    out = ['', f'ns_phase_kernel MFMA counters ({max(len(util), len(rate))} dispatches; {simds} SIMDs, '
               f'{xcc} XCDs, max engine clock {fmax:.0f} MHz):']
    if util:
        out.append(f'- MFMA busy (MfmaUtil): {100 * avg(util):.1f}% (min {100 * min(util):.1f}%, '
                   f'max {100 * max(util):.1f}%); shader clock while busy {avg(clk):.2f} GHz')
    if rate:
        out.append(f'- executed f16 MFMA flops: {avg(rate):.0f} TFLOP/s per dispatch on average')
    return out


def vendor_gemm() -> int:
    """The vendor library on the same products as full (unsymmetric) GEMMs: torch.bmm in f16 over
    the config-2 shapes (hipBLASLt/rocBLAS), and two square GEMMs for scale. One JSON line."""
    import torch
    dev = torch.device('cuda:0')
    g = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape):
        return torch.randn(*shape, device=dev, dtype=torch.float16, generator=g)

    def t(fn, flops, iters=20):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / iters
        return {'ms': round(dt * 1e3, 4), 'tflops': round(flops / dt / 1e12, 1)}

    res = {}
    for n in (4096, 8192):
        a, b = rnd(n, n), rnd(n, n)
        res[f'mm_{n}'] = t(lambda: a @ b, 2.0 * n ** 3)
        del a, b
    a, b = rnd(140, 1024, 1024), rnd(140, 1024, 1024)
    res['bmm_140x1024^3'] = t(lambda: torch.bmm(a, b), 140 * 2.0 * 1024 ** 3)
    x = rnd(60, 1024, 3072)
    xt = x.transpose(1, 2).contiguous()
    res['bmm_60x(1024x3072)(3072x1024)'] = t(lambda: torch.bmm(x, xt), 60 * 2.0 * 1024 * 1024 * 3072)
    res['bmm_60x(1024x1024)(1024x3072)'] = t(lambda: torch.bmm(a[:60], x), 60 * 2.0 * 1024 * 1024 * 3072)
    print(json.dumps({'vendor_gemm_f16': res, 'peak_tflops': MFMA_PEAK_TFLOPS}), flush=True)
    return 0


def traffic_from_profile(kernel: str) -> float | None:
    """HBM bytes per launch of `kernel` from its committed counter summary, if present."""
    import re
    if kernel not in TRAFFIC_PROFILES:
        return None
    try:
        text = open(os.path.join(ROOT, 'profiles', TRAFFIC_PROFILES[kernel])).read()
    except OSError:
        return None
    m = re.search(kernel + r' HBM bytes per launch: ([0-9.eE+]+)', text)
    return float(m.group(1)) if m else None


# ---------------------------------------------------------------------------------------------
# GPU measurement
# ---------------------------------------------------------------------------------------------

def time_launches(torch, thorn_amd, opt, one_step, steps: int):
    """Runs `steps` steps with a HIP event pair around every launch of opt's plans. Orthogonalized
    plans report each launch's start and end (a large group runs as chains on several streams whose
    launches overlap); Adam plans their summed durations. Returns kind -> (summed ms, launches),
    kind -> [(start ms, end ms)] and kind -> summed ms of the plans without intervals."""
    plans = [pl for r in opt._runners.values() for pl in r.plans]
    for pl in plans:
        pl.timing_enable(64 * steps)
    ref = torch.cuda.Event(enable_timing=True)
    ref.record()
    for _ in range(steps):
        one_step()
    torch.cuda.synchronize()
    kinds: dict = {}
    intervals: dict = {}
    summed: dict = {}
    for pl in plans:
        if isinstance(pl, thorn_amd._lib.OrthoPlan):
            for k, a, b in pl.timing_intervals(ref.cuda_event, 64 * steps):
                tot, cnt = kinds.get(k, (0.0, 0))
                kinds[k] = (tot + (b - a), cnt + 1)
                intervals.setdefault(k, []).append((a, b))
        else:
            for k, (ms, n) in pl.timing_read().items():
                tot, cnt = kinds.get(k, (0.0, 0))
                kinds[k] = (tot + ms, cnt + n)
                summed[k] = summed.get(k, 0.0) + ms
        pl.timing_enable(0)
    return kinds, intervals, summed


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--config', type=int, default=2)
    ap.add_argument('--momentum-align', action='store_true',
                    help='Magma on every group (a variant of the workload, not the headline line: masked '
                         'matrices skip Newton-Schulz, so the per-launch flops vary and no roofline is given)')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument('--cpu-budget', type=float, default=300.0,
                    help='seconds of oracle time on the host for cpu_baseline (config 2: every shape fits)')
    ap.add_argument('--polar-decomp-batch-size', type=int, default=None,
                    help="elements per Newton-Schulz batch (the optimizer's polar_decomp_batch_size; "
                         "default: the library's, one batch per group)")
    ap.add_argument('--single-chain', action='store_true',
                    help='step the orthogonalized group as one plan on one stream (the library default splits '
                         'a large group into two chains on two streams)')
    ap.add_argument('--no-one-chain', action='store_true',
                    help='skip the one-plan pass behind roofline.one_chain (kernel traces: that pass runs on '
                         'the caller\'s stream after the chained steps)')
    ap.add_argument('--per-param', action='store_true',
                    help='step each parameter on its own, as gradient release does from its hook (a '
                         'variant of the workload, not the headline line: step time only, no roofline)')
    ap.add_argument('--in-order', action='store_true',
                    help='with --per-param: every step on the caller\'s stream, in order')
    ap.add_argument('--release-window-mib', type=float, default=None,
                    help='with --per-param: gradient bytes per gradient-release window (the library\'s '
                         'RELEASE_WINDOW_BYTES; 0: each parameter alone)')
    ap.add_argument('--copy-cal-mib', type=int, default=0,
                    help='run one torch.neg over this many MiB first (counter calibration)')
    ap.add_argument('--vendor-gemm', action='store_true',
                    help='time torch (hipBLASLt) f16 GEMMs of the Newton-Schulz shapes for comparison and exit')
    ap.add_argument('--rocprof-summary', metavar='DIR', nargs='+',
                    help='print a markdown summary of rocprofv3 CSV output directories and exit')
    args = ap.parse_args()
    if args.rocprof_summary:
        print(rocprof_summary(args.rocprof_summary, args.copy_cal_mib, args.steps, args.config))
        return 0
    if args.vendor_gemm:
        return vendor_gemm()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one MI355X: this build has no multi-GPU path (each matrix\'s step '
              'is independent, so a group would shard by whole matrices). Run with --gpus 1.', file=sys.stderr)
        return 2

    import torch
    import thorn_amd

    if args.single_chain:
        thorn_amd.optim.CHAIN_MIN_MATRICES = 1 << 30
    if args.in_order:
        thorn_amd.optim.RELEASE_OVERLAP = False
    if args.release_window_mib is not None:
        thorn_amd.optim.RELEASE_WINDOW_BYTES = int(args.release_window_mib * (1 << 20))
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    if args.copy_cal_mib:
        copy_calibration(args.copy_cal_mib, dev)
    t0 = time.perf_counter()
    params, grads, groups, mats = build_workload(args.config, dev)
    if args.momentum_align:
        for g in groups:
            g['momentum_align'] = True
    gen_s = time.perf_counter() - t0
    n_m = len(mats)
    opt = thorn_amd.THORN(groups)
    if args.polar_decomp_batch_size is not None:
        opt.polar_decomp_batch_size = args.polar_decomp_batch_size

    def one_step():
        if args.per_param:   # gradient release: each parameter's step once its gradient is there,
            for p, g in zip(params, grads):   # as the hooks run it, joined as at the end of backward
                p.grad = g
                opt._release_step(p, join_later=True)
            opt._release_join()
            return
        for p, g in zip(params, grads):
            p.grad = g
        opt.step()

    t0 = time.perf_counter()
    one_step()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1000.0
    for _ in range(max(0, args.warmup - 1)):
        one_step()
    torch.cuda.synchronize()

    # timed region: exactly K steps
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        one_step()
    ev1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    gpu_ms = ev0.elapsed_time(ev1) / args.steps

    if args.per_param:   # one plan per parameter: step time only
        print(json.dumps({
            'metric': 'THORN step ms with gradient release (opt.step(param=p) for each parameter), 1 GPU',
            'value': round(wall_ms, 3), 'unit': 'ms', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
            'ms_per_step': round(wall_ms, 3), 'higher_is_better': False, 'scaling': 'weak', 'vs_baseline': None,
            'dtype': 'f16', 'data': 'synthetic',
            'config': {'workload': f'config {args.config}, per-parameter steps'
                       + (' in order' if args.in_order else
                          f' (large ones in windows of {thorn_amd.optim.RELEASE_WINDOW_BYTES >> 20} MiB of gradients '
                          'on the release streams)'), 'matrices': n_m,
                       'adam_tensors': len(params) - n_m},
            'gpu_event_ms_per_step': round(gpu_ms, 3), 'first_step_ms': round(first_ms, 1),
            'runners': len(opt._runners), 'roofline': None, 'cpu_baseline': None}), flush=True)
        return 0

    # per-kernel breakdown: the same K steps again with a HIP event pair around every launch
    kinds, intervals, summed = time_launches(torch, thorn_amd, opt, one_step, args.steps)

    def union_ms(names) -> float:
        """The union of the launch intervals of the given kernel kinds, plus their summed durations
        in plans timed without intervals."""
        return (_union_us([x for k in names for x in intervals.get(k, [])])
                + sum(summed.get(k, 0.0) for k in names))

    grp0 = thorn_amd.optim._Group.from_kwargs(**opt.param_groups[0])
    mask = thorn_amd.optim._OrthoRunner.restart_mask(grp0, grp0.iters)
    F = schedule_flops(mats, grp0.iters, mask)
    small = [sh for sh in mats if min(sh) <= SMALL_MAX_S and sh[0] * sh[1] < SMALL_MAX_ELEMS]
    F_small = schedule_flops(small, grp0.iters, mask)
    ns_ms = union_ms(NS_KINDS) / args.steps
    upd_ms = union_ms(('pre', 'norm', 'rowstats', 'pnn_apply', 'adam')) / args.steps
    cbytes = compulsory_bytes(mats, params, n_m)
    # dominant kernel: ns_phase_kernel, which runs the Newton-Schulz products of the large
    # matrices (one launch per schedule step); with no large matrix, ns_small_kernel. Its
    # algorithmic flops per launch are its matrices' schedule flops over its launch count.
    if F - F_small > 0:
        dom_kinds = ('gram', 'poly', 'symprod', 'update')
        dom_name, dom_flops = 'ns_phase_kernel', F - F_small
    else:
        dom_kinds, dom_name, dom_flops = ('small',), 'ns_small_kernel', F_small
    ns_launches = sum(kinds.get(k, (0.0, 0))[1] for k in NS_KINDS) / args.steps
    dom_launches = sum(kinds.get(k, (0.0, 0))[1] for k in dom_kinds) / args.steps
    dom_ms = union_ms(dom_kinds) / args.steps
    dom_sum_ms = sum(kinds.get(k, (0.0, 0))[0] for k in dom_kinds) / args.steps
    ns_flops_per_launch = dom_flops / max(dom_launches, 1)
    # the dominant kernel's time per launch: the union of its launch intervals per launch (its
    # launches of two chains overlap one another)
    u_avg = dom_ms / max(dom_launches, 1)
    achieved = ns_flops_per_launch / (u_avg * 1e-3) / 1e12 if u_avg > 0 else 0.0
    chains = max([len(r.plans) if getattr(r, 'chained', False) else 1 for r in opt._runners.values()] + [1])
    # With chains, the dominant kernel's launches share the chip with one another and with the
    # other chains' memory-bound kernels. The same step as one plan on one stream (a second
    # optimizer over the same parameters, after every figure above is taken) gives its rate alone.
    one_chain = upd_one = None
    if chains > 1 and not args.momentum_align and not args.no_one_chain:
        keep = thorn_amd.optim.CHAIN_MIN_MATRICES
        thorn_amd.optim.CHAIN_MIN_MATRICES = 1 << 30
        try:
            opt1 = thorn_amd.THORN(groups)

            def step1():
                for p, g in zip(params, grads):
                    p.grad = g
                opt1.step()
            for _ in range(max(3, args.warmup)):
                step1()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record()
            for _ in range(args.steps):
                step1()
            e1.record()
            torch.cuda.synchronize()
            k1, iv1, su1 = time_launches(torch, thorn_amd, opt1, step1, args.steps)
            d1 = (_union_us([x for k in dom_kinds for x in iv1.get(k, [])])
                  + sum(su1.get(k, 0.0) for k in dom_kinds)) / args.steps
            n1 = sum(k1.get(k, (0.0, 0))[1] for k in dom_kinds) / args.steps
            a1 = dom_flops / (d1 * 1e-3) / 1e12 if d1 > 0 else 0.0
            # the update kernels alone: on one stream (no chains, no Adam side stream) nothing
            # overlaps them, so the union of their intervals is their own time
            uk = ('pre', 'norm', 'rowstats', 'pnn_apply', 'adam')
            upd1 = (_union_us([x for k in uk for x in iv1.get(k, [])]) + sum(su1.get(k, 0.0) for k in uk)) / args.steps
            if upd1 > 0:
                upd_one = {'ms_per_step': round(upd1, 3), 'gbps': round(cbytes / (upd1 * 1e-3) / 1e9, 1),
                           'hbm_frac': round(cbytes / (upd1 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
            one_chain = {'gpu_ms_per_step': round(e0.elapsed_time(e1) / args.steps, 3), 'achieved': round(a1, 1),
                         'frac': round(a1 / MFMA_PEAK_TFLOPS, 4), 'launches_per_step': n1,
                         'avg_launch_ms': round(d1 / max(n1, 1), 4)}
            del opt1
        finally:
            thorn_amd.optim.CHAIN_MIN_MATRICES = keep
    phases = {k: {'ms_per_launch': round(ms / n, 4), 'launches_per_step': n / args.steps}
              for k, (ms, n) in sorted(kinds.items())}

    cpu = None if (args.no_cpu_baseline or args.momentum_align) else cpu_baseline(args.config, args.cpu_budget)
    ms = wall_ms
    out = {
        'metric': 'THORN step ms, 300M Qwen3 param set, 1 GPU; NS TFLOP/s and % MFMA peak',
        'value': round(ms, 3),
        'unit': 'ms',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms, 3),
        'higher_is_better': False,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f16',
        'data': 'synthetic',
        'config': {'workload': {1: 'one 512x256 Linear (config 1)', 2: 'qwen3-300m (BASELINE config 2)', 3: 'qwen3-300m decouple_md (config 3)',
                                4: 'earshot conv VAD (config 4)', 5: 'qwen3-1.7b matrices (config 5)'}[args.config]
                   + (' + Magma momentum_align' if args.momentum_align else ''),
                   'matrices': n_m, 'adam_tensors': len(params) - n_m,
                   'ortho_elements': sum(r * c for r, c in mats),
                   'adam_elements': sum(p.numel() for p in params[n_m:]), 'ns_iters': 5,
                   'polar_decomp_batch_size': opt.polar_decomp_batch_size,
                   'workspace_bytes': sum({ws.data_ptr(): ws.numel() for r in opt._runners.values()
                                           for ws in r.workspaces}.values()),
                   'ns_arith': 'f16 MFMA, fp32 accumulate; fp32 state'},
        'gpu_event_ms_per_step': round(gpu_ms, 3),
        'first_step_ms': round(first_ms, 1),
        'ns': {'schedule': {'square': op_counts(plain_ops(grp0.iters)),
                            'other': op_counts(gram_ops(grp0.iters, mask)), 'restart_mask': mask},
               'flops_per_step': F,
               'plain_quintic_flops': ns_flops(mats), 'ms_per_step': round(ns_ms, 3),
               'tflops': round(F / (ns_ms * 1e-3) / 1e12, 1) if ns_ms > 0 else None,
               'mfma_frac': round(F / (ns_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4) if ns_ms > 0 else None},
        'update': {'compulsory_bytes': cbytes, 'ms_per_step': round(upd_ms, 3),
                   'gbps': round(cbytes / (upd_ms * 1e-3) / 1e9, 1) if upd_ms > 0 else None,
                   'hbm_frac': round(cbytes / (upd_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4) if upd_ms > 0 else None,
                   'one_chain': upd_one},
        'roofline': {'kernel': dom_name, 'bound': 'mfma', 'achieved': round(achieved, 1),
                     'peak': MFMA_PEAK_TFLOPS, 'unit': 'TFLOP/s', 'frac': round(achieved / MFMA_PEAK_TFLOPS, 4),
                     'traffic': traffic_from_profile(dom_name), 'flops_per_launch': ns_flops_per_launch,
                     'launches_per_step': dom_launches, 'avg_launch_ms': round(u_avg, 4),
                     'active_ms_per_step': round(dom_ms, 3), 'launch_ms_sum_per_step': round(dom_sum_ms, 3),
                     'chains': chains, 'one_chain': one_chain},
        'launches_per_step': {'ns': ns_launches,
                              'total': sum(n for _, n in kinds.values()) / args.steps},
        'phases': phases,
        'cpu_baseline': cpu,
        'workload_gen_s': round(gen_s, 1),
    }
    if args.momentum_align:   # NS flops depend on which matrices each step's masks applied
        out['roofline'] = None
        out['ns'] = {'ms_per_step': round(ns_ms, 3), 'launches_per_step': ns_launches}
    print(json.dumps(out), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
