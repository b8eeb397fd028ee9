"""The Newton-Schulz block map (thorn_amd/csrc/task_layout.hpp), compiled for the host with g++:
every (matrix, tile) lands on exactly one position; the positions xcd_split gives each XCD (eight
contiguous chunks) hold an equal share of every matrix with more tiles than half a chunk, as a
contiguous range of its tiles at the front of the chunk; lists without such a matrix keep the
plain order (each matrix whole, in list order)."""
from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HDR = ROOT / 'thorn_amd' / 'csrc' / 'task_layout.hpp'


@pytest.fixture(scope='module')
def layout(tmp_path_factory):
    gxx = shutil.which('g++')
    if gxx is None:
        pytest.skip('g++ not available')
    d = tmp_path_factory.mktemp('layout')
    src = d / 'l.cpp'
    src.write_text(f'#include "{HDR}"\n'
                   'extern "C" int write_map(int32_t* m, const int32_t* o, int n, const int64_t* b) {\n'
                   '    return thorn_layout::write_block_map(m, o, n, b) ? 1 : 0;\n}\n'
                   'extern "C" long cluster_map(int32_t* m, const int32_t* l, int n, const int64_t* c, int32_t* s) {\n'
                   '    return static_cast<long>(thorn_layout::write_cluster_map(m, l, n, c, s));\n}\n')
    so = d / 'l.so'
    res = subprocess.run([gxx, '-O2', '-std=c++17', '-shared', '-fPIC', str(src), '-o', str(so)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    lib = ctypes.CDLL(str(so))
    lib.write_map.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int, ctypes.c_void_p]
    lib.write_map.restype = ctypes.c_int
    lib.cluster_map.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_int] + [ctypes.c_void_p] * 2
    lib.cluster_map.restype = ctypes.c_long

    def run(order, blocks):
        order = np.asarray(order, dtype=np.int32)
        blocks = np.asarray(blocks, dtype=np.int64)
        total = int(blocks[order].sum())
        m = np.full(2 * max(total, 1), -1, dtype=np.int32)
        assert lib.write_map(m.ctypes.data, order.ctypes.data, len(order), blocks.ctypes.data) == 1
        return m[:2 * total].reshape(total, 2)

    def clusters(live, cluster_of):
        live = np.asarray(live, dtype=np.int32)
        cluster_of = np.asarray(cluster_of, dtype=np.int64)
        cap = 8 * int(cluster_of[live].sum()) if len(live) else 8
        m = np.full(2 * max(cap, 1), -7, dtype=np.int32)
        srt = np.zeros(max(len(live), 1), dtype=np.int32)
        grid = lib.cluster_map(m.ctypes.data, live.ctypes.data, len(live), cluster_of.ctypes.data, srt.ctypes.data)
        assert 0 <= grid <= cap and grid % 8 == 0
        assert (m[2 * grid:] == -7).all()   # nothing written past the grid
        return grid, m[:2 * grid].reshape(grid, 2)
    run.clusters = clusters
    return run


def chunks(total):
    pp, rp = divmod(total, 8)
    out, s = [], 0
    for j in range(8):
        c = pp + (1 if j < rp else 0)
        out.append((s, s + c))
        s += c
    return out


def test_bijection_and_striping(layout):
    rng = np.random.default_rng(3)
    for case in range(300):
        n = int(rng.integers(1, 40))
        blocks = rng.integers(1, 60, size=n)
        for _ in range(int(rng.integers(0, 4))):              # a few big matrices
            blocks[rng.integers(0, n)] = int(rng.integers(60, 3000))
        order = rng.permutation(n)
        m = layout(order, blocks)
        total = int(blocks.sum())
        pairs = {(int(a), int(b)) for a, b in m}
        assert len(pairs) == total
        assert pairs == {(int(i), t) for i in range(n) for t in range(int(blocks[i]))}
        big = max(16, (total // 8) // 2)
        if blocks[blocks > big].sum() > total // 2:
            continue   # the striped matrices fill most chunks: parts move to where there is room
        for i in range(n):
            if blocks[i] <= big:
                continue
            for lo, hi in chunks(total):
                tiles = [int(t) for a, t in m[lo:hi] if a == i]
                assert tiles == list(range(tiles[0], tiles[0] + len(tiles))) if tiles else True
                assert abs(len(tiles) - blocks[i] / 8) <= 2, (case, i, len(tiles), blocks[i])


def test_plain_order_without_big_matrices(layout):
    """Config 2's lists (10 to 48 tiles per matrix, 140 matrices): the map is the list order."""
    blocks = np.array([10] * 40 + [16] * 20 + [24] * 40 + [48] * 40)
    order = np.random.default_rng(1).permutation(len(blocks))
    m = layout(order, blocks)
    want = [(int(i), t) for i in order for t in range(int(blocks[i]))]
    assert [tuple(map(int, r)) for r in m] == want


def test_config5_big_matrix_spread(layout):
    """One 8192 x 8192 matrix (1024 update tiles) beside 27 smaller ones: each XCD's chunk starts
    with its eighth of the big matrix's tiles."""
    blocks = np.array([1024] + [64] * 27)
    m = layout(np.arange(28), blocks)
    for lo, hi in chunks(int(blocks.sum())):
        assert (m[lo:lo + 128, 0] == 0).all() and (m[lo + 128:hi, 0] != 0).all()


def test_small_cluster_map(layout):
    """ns_small_kernel's block map (write_cluster_map): every (matrix, member) of the live list on
    exactly one block, a cluster's members on consecutive blocks of one residue mod 8 (block b runs
    on XCD b mod 8), the clusters dealt largest first to the XCD with the fewest blocks, blocks past
    an XCD's share idle (-1), and the grid 8 times the largest share."""
    rng = np.random.default_rng(11)
    # config 4's seven matrices: clusters 1, 1, 1, 1, 1, 10, 1
    grid, m = layout.clusters(list(range(7)), [1, 1, 1, 1, 1, 10, 1])
    assert grid == 80
    assert [int(b) for b in np.nonzero(m[:, 0] == 5)[0]] == [8 * j for j in range(10)]
    for case in range(300):
        n = int(rng.integers(1, 30))
        cluster_of = rng.choice([1, 1, 1, 4, 6, 10, 16], size=n)
        live = sorted(rng.choice(n, size=int(rng.integers(1, n + 1)), replace=False).tolist())
        grid, m = layout.clusters(live, cluster_of)
        share = [0] * 8
        seen = {}
        for b, (mat, mc) in enumerate(m):
            if mat == -1:
                assert mc == 0
                continue
            member, c = int(mc) & 255, int(mc) >> 8
            assert c == cluster_of[mat] and (int(mat), member) not in seen, (case, b)
            seen[(int(mat), member)] = b
            share[b % 8] += 1
        assert set(seen) == {(i, j) for i in live for j in range(int(cluster_of[i]))}, case
        for i in live:
            blocks = [seen[(i, j)] for j in range(int(cluster_of[i]))]
            assert len({b % 8 for b in blocks}) == 1, (case, i, blocks)
            assert [b // 8 for b in blocks] == list(range(blocks[0] // 8, blocks[0] // 8 + len(blocks)))
        assert grid == 8 * max(share)
        # greedy by size: the shares differ by at most the largest cluster
        assert max(share) - min(share) <= max(int(cluster_of[i]) for i in live), (case, share)
