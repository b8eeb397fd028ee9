// Block map of a Newton-Schulz task list (host code, shared by thorn_abi.hip and its CPU test).
//
// ns_phase_kernel's blocks find their (matrix, tile) in a per-block map, and xcd_split gives each
// XCD a contiguous chunk of the list's positions: chunk j holds positions
// [j * pp + min(j, rp), ...) of size pp + (j < rp), pp = total / 8, rp = total % 8, and an XCD runs
// its chunk in position order. Matrices come in the list's order (dealt to 8 bins by cost); a
// matrix stays whole on one XCD, so the tiles that share its operand panels share an L2.
//
// A matrix with more tiles than half a chunk would hold one XCD long after the others are done
// (config 5's 8192 x 8192 matrix: its 1024 update tiles of K = 8192 kept ~60 of 256 CUs busy for
// ~2.4 ms per launch while the rest idled). Such a matrix is striped: its tiles, in order, are cut
// into 8 contiguous parts, one per chunk, placed at the front of each chunk (the long tiles first),
// largest striped matrix first. The other matrices then fill the chunks in list order, as before.
// Every position receives exactly one tile; nothing is allocated (fill_table runs every step).
#pragma once
#include <algorithm>
#include <stdint.h>
#include <utility>

namespace thorn_layout {

// m: 2 * total int32 (matrix, tile) pairs; order: the list's matrices; blocks_of[i]: tiles of
// matrix i. Returns false if the map could not be filled (never for consistent inputs).
inline bool write_block_map(int32_t* m, const int32_t* order, int n, const int64_t* blocks_of) {
    int64_t total = 0;
    for (int k = 0; k < n; ++k) total += blocks_of[order[k]];
    const int64_t pp = total / 8, rp = total % 8;
    int64_t cap[8], start[8], fill[8];
    for (int j = 0; j < 8; ++j) {
        cap[j] = pp + (j < rp ? 1 : 0);
        start[j] = j * pp + std::min<int64_t>(j, rp);
        fill[j] = 0;
    }
    auto put = [&](int j, int32_t mat, int64_t tile) {
        const int64_t pos = start[j] + fill[j]++;
        m[2 * pos] = mat;
        m[2 * pos + 1] = static_cast<int32_t>(tile);
    };
    // striped matrices: more tiles than half a chunk (and at least 16), up to 64 of them
    constexpr int kMaxStriped = 64;
    int striped[kMaxStriped];
    int ns = 0;
    const int64_t big = std::max<int64_t>(16, pp / 2);
    for (int k = 0; k < n && ns < kMaxStriped; ++k)
        if (blocks_of[order[k]] > big) striped[ns++] = k;
    std::stable_sort(striped, striped + ns,
                     [&](int a, int b) { return blocks_of[order[a]] > blocks_of[order[b]]; });
    for (int s = 0; s < ns; ++s) {
        const int32_t mat = order[striped[s]];
        const int64_t T = blocks_of[mat];
        int64_t tile = 0, carry = 0;
        for (int j = 0; j < 8; ++j) {
            const int64_t want = T / 8 + (j < T % 8 ? 1 : 0) + carry;
            const int64_t take = std::min(want, cap[j] - fill[j]);
            for (int64_t q = 0; q < take; ++q) put(j, mat, tile++);
            carry = want - take;
        }
        for (int j = 0; j < 8 && tile < T; ++j)   // what no chunk had room for in turn
            while (tile < T && fill[j] < cap[j]) put(j, mat, tile++);
        if (tile < T) return false;
    }
    // the others, whole, in list order, chunk after chunk
    int j = 0;
    for (int k = 0; k < n; ++k) {
        bool is_striped = false;
        for (int s = 0; s < ns; ++s) is_striped = is_striped || striped[s] == k;
        if (is_striped) continue;
        const int32_t mat = order[k];
        for (int64_t tile = 0; tile < blocks_of[mat]; ++tile) {
            while (j < 8 && fill[j] == cap[j]) ++j;
            if (j == 8) return false;
            put(j, mat, tile);
        }
    }
    return true;
}

// Block map of ns_small_kernel: each matrix's cluster of workgroups (cluster_of[i] of them) on
// one XCD. Block b runs on XCD b mod 8, so a cluster takes blocks of one residue x, x + 8 j for
// consecutive j; clusters are dealt largest first (stable) to the XCD with the fewest blocks (the
// lowest x on a tie). m[2b] = matrix, m[2b + 1] = member | C << 8, or m[2b] = -1 for a block past
// its XCD's share. sorted: room for n entries (no allocation: fill_table runs every step). Returns
// the launch's block count, 8 times the largest share; m needs 2 * 8 * sum(cluster_of) entries.
inline int64_t write_cluster_map(int32_t* m, const int32_t* list, int n, const int64_t* cluster_of, int32_t* sorted) {
    for (int k = 0; k < n; ++k) sorted[k] = list[k];
    for (int a = 1; a < n; ++a)   // insertion sort by cluster size, stable
        for (int b = a; b > 0 && cluster_of[sorted[b]] > cluster_of[sorted[b - 1]]; --b) std::swap(sorted[b], sorted[b - 1]);
    int64_t fill[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int k = 0; k < n; ++k) {
        const int32_t i = sorted[k];
        int x = 0;
        for (int y = 1; y < 8; ++y)
            if (fill[y] < fill[x]) x = y;
        const int64_t C = cluster_of[i];
        for (int64_t j = 0; j < C; ++j) {
            const int64_t b = x + 8 * (fill[x] + j);
            m[2 * b] = i;
            m[2 * b + 1] = static_cast<int32_t>(j | (C << 8));
        }
        fill[x] += C;
    }
    int64_t most = 0;
    for (int x = 0; x < 8; ++x) most = std::max(most, fill[x]);
    for (int x = 0; x < 8; ++x)
        for (int64_t j = fill[x]; j < most; ++j) {
            m[2 * (x + 8 * j)] = -1;
            m[2 * (x + 8 * j) + 1] = 0;
        }
    return 8 * most;
}

}  // namespace thorn_layout
